"""Wrapper formats the reference does not decode: gzip, raw DEFLATE, preset dictionaries.

Valid streams must decode bit-exactly as CPU zlib decodes them
(``zlib.decompress`` with wbits 31 and -15, ``decompressobj(zdict=...)``), on
both routes (outputs up to 64 KiB take the one-wave route, larger ones the
parallel one).  The statuses of broken wrappers are this codec's own
(24: gzip CRC-32/ISIZE, 25: dictionary DICTID; the rest as for zlib streams),
checked case by case.  The drop-in zlib calls keep the reference's refusals
(16 for gzip, 17 for FDICT without a dictionary).
"""

import gzip
import struct
import zlib

import numpy as np
import pytest

import workloads

pytestmark = pytest.mark.gpu

SIZES = [0, 1, 4000, 65536, 65537, 300000, 3 << 20]


def _text(n, seed=0):
    return workloads.text_like(n, np.random.default_rng(seed))


def _raw_deflate(data, level=6, zdict=None, strategy=zlib.Z_DEFAULT_STRATEGY):
    kwargs = {"zdict": zdict} if zdict is not None else {}
    c = zlib.compressobj(level, zlib.DEFLATED, -15, 8, strategy, **kwargs)
    return c.compress(data) + c.flush()


def _gzip_member(data, *, extra=None, name=None, comment=None, hcrc=False, level=6):
    flags = (4 if extra is not None else 0) | (8 if name is not None else 0) | \
        (16 if comment is not None else 0) | (2 if hcrc else 0)
    header = bytes((0x1F, 0x8B, 8, flags)) + struct.pack("<I", 12345) + bytes((0, 3))
    if extra is not None:
        header += struct.pack("<H", len(extra)) + extra
    if name is not None:
        header += name + b"\0"
    if comment is not None:
        header += comment + b"\0"
    if hcrc:
        header += struct.pack("<H", zlib.crc32(header) & 0xFFFF)
    trailer = struct.pack("<II", zlib.crc32(data), len(data) & 0xFFFFFFFF)
    return header + _raw_deflate(data, level) + trailer


def _status(meta):
    return int(meta.cpu().numpy()[0])


@pytest.mark.parametrize("size", SIZES)
def test_gzip_from_the_standard_library(gpu, no_cpu_codec, size):
    import cuda_zlib
    data = _text(size, size)
    stream = gzip.compress(data, 6, mtime=0)
    with no_cpu_codec:
        out = cuda_zlib.decompress_gzip(stream, size, 0)
    assert out.cpu().numpy().tobytes() == data


@pytest.mark.parametrize("fields", ["extra", "name", "comment", "hcrc", "all"])
@pytest.mark.parametrize("size", [5000, 200000])
def test_gzip_optional_header_fields(gpu, no_cpu_codec, fields, size):
    import cuda_zlib
    data = workloads.strain(size // 4, 5)
    kwargs = {"extra": b"BC\x02\x00\x10\x00", "name": b"strain.f32", "comment": b"seeded",
              "hcrc": True}
    if fields != "all":
        kwargs = {fields: kwargs[fields]}
    stream = _gzip_member(data, **kwargs)
    assert zlib.decompress(stream, 31) == data
    with no_cpu_codec:
        out, meta = cuda_zlib.decompress_gzip_checked(stream, len(data), 0)
        assert _status(meta) == 0
    assert out.cpu().numpy().tobytes() == data


def _gzip_cases():
    data = _text(100000, 3)
    good = _gzip_member(data, name=b"x", hcrc=True)
    small = _gzip_member(data[:3000])
    bad_crc = good[:-8] + struct.pack("<I", zlib.crc32(data) ^ 1) + good[-4:]
    bad_isize = good[:-4] + struct.pack("<I", len(data) + 1)
    bad_hcrc = bytearray(good)
    bad_hcrc[12] ^= 0x01  # inside the name: the header CRC no longer matches
    return [
        ("crc-general", bad_crc, len(data), 24, data),
        ("isize-general", bad_isize, len(data), 24, data),
        ("crc-small", small[:-8] + struct.pack("<I", zlib.crc32(data[:3000]) ^ 4) + small[-4:],
         3000, 24, data[:3000]),
        ("header-crc", bytes(bad_hcrc), len(data), 15, None),
        ("magic", b"\x1f\x8c" + good[2:], len(data), 15, None),
        ("method", good[:2] + b"\x07" + good[3:], len(data), 15, None),
        ("reserved-flag", good[:3] + bytes((good[3] | 0x20,)) + good[4:], len(data), 15, None),
        ("truncated-wrapper", good[:17], 0, 14, None),
        # FNAME set, but its terminating zero never comes before the trailer.
        ("name-runs-into-trailer", bytes((0x1F, 0x8B, 8, 8)) + bytes(6) + b"abcdefgh", 0, 14, None),
        ("second-member", small + small, 3000, 12, None),
        ("size-short", good, len(data) - 1, 7, None),
    ]


def test_gzip_long_header_fields_on_the_general_route(gpu, no_cpu_codec):
    """A 300 KB FNAME, a comment and FHCRC before a 200 KB body: the general
    route's frame pass finds the terminators and the header CRC-32 with its
    whole workgroup, with parse_frame's statuses (0, 15 for a header CRC that
    does not match, 14 for a name that runs into the trailer)."""
    import cuda_zlib
    data = _text(200000, 41)
    name = bytes(np.random.default_rng(42).integers(1, 256, 300000, dtype=np.uint8))
    good = _gzip_member(data, name=name, comment=b"c" * 5000, hcrc=True)
    assert zlib.decompress(good, 31) == data
    bad_hcrc = bytearray(good)
    bad_hcrc[150000] = 1 if bad_hcrc[150000] != 1 else 2  # inside the name, still not zero
    runs_on = bytes((0x1F, 0x8B, 8, 8)) + bytes(6) + name + bytes(8)  # no zero before the trailer
    for stream, status in ((good, 0), (bytes(bad_hcrc), 15), (runs_on, 14)):
        with no_cpu_codec:
            out, meta = cuda_zlib.decompress_gzip_checked(stream, len(data), 0)
            assert _status(meta) == status
        got = out.cpu().numpy().tobytes()
        assert got == (data if status == 0 else bytes(len(data)))


@pytest.mark.parametrize("case", _gzip_cases(), ids=lambda c: c[0])
def test_gzip_wrapper_failures(gpu, no_cpu_codec, case):
    import cuda_zlib
    _, stream, expected, status, keep = case
    with no_cpu_codec:
        out, meta = cuda_zlib.decompress_gzip_checked(stream, expected, 0)
        got = _status(meta)
    assert got == status
    data = out.cpu().numpy().tobytes()
    # A checksum mismatch keeps the decoded bytes (as zlib's Adler-32 status 21
    # does); every other failure of the parallel route leaves zeros.
    if keep is not None:
        assert data == keep
    elif expected > 65536:
        assert data == bytes(expected)


@pytest.mark.parametrize("size", SIZES)
@pytest.mark.parametrize("level", [1, 9])
def test_raw_deflate(gpu, no_cpu_codec, size, level):
    import cuda_zlib
    data = _text(size, 7 + size)
    stream = _raw_deflate(data, level)
    with no_cpu_codec:
        out = cuda_zlib.decompress_deflate_raw(stream, size, 0)
    assert out.cpu().numpy().tobytes() == data


def test_raw_deflate_failures(gpu, no_cpu_codec):
    import cuda_zlib
    data = _text(120000, 8)
    stream = _raw_deflate(data)
    with no_cpu_codec:
        _, meta = cuda_zlib.decompress_deflate_raw_checked(stream + b"\x00", len(data), 0)
        assert _status(meta) == 12  # a byte after the final block
        _, meta = cuda_zlib.decompress_deflate_raw_checked(stream[:-3], len(data), 0)
        assert _status(meta) != 0
        _, meta = cuda_zlib.decompress_deflate_raw_checked(b"", 0, 0)
        assert _status(meta) == 1


def _dictionary(n, seed):
    return _text(n, seed)


@pytest.mark.parametrize("size", [1, 5000, 65536, 200000, 2 << 20])
@pytest.mark.parametrize("dict_size", [100, 32768, 50000])
def test_zlib_preset_dictionary(gpu, no_cpu_codec, size, dict_size):
    import cuda_zlib
    zdict = _dictionary(dict_size, 11)
    # Data that repeats dictionary text, so that references reach into it.
    data = (zdict[-20000:] + _text(size, 12))[:size]
    c = zlib.compressobj(6, zlib.DEFLATED, 15, 8, zlib.Z_DEFAULT_STRATEGY, zdict=zdict)
    stream = c.compress(data) + c.flush()
    assert stream[1] & 0x20  # the header asks for the dictionary
    d = zlib.decompressobj(zdict=zdict)
    assert d.decompress(stream) == data
    with no_cpu_codec:
        out = cuda_zlib.decompress_zlib(stream, size, 0, zdict=zdict)
        assert out.cpu().numpy().tobytes() == data
        _, meta = cuda_zlib.decompress_zlib_checked(stream, size, 0, zdict=zdict[:-1] + b"?")
        assert _status(meta) == 25
        with pytest.raises(cuda_zlib.UnsupportedStream):
            cuda_zlib.decompress_zlib(stream, size, 0)  # the reference's refusal stands


@pytest.mark.parametrize("size", [3000, 65537, 500000])
def test_raw_deflate_with_history(gpu, no_cpu_codec, size):
    import cuda_zlib
    zdict = _dictionary(40000, 13)
    data = (zdict[5000:30000] + _text(size, 14))[:size]
    stream = _raw_deflate(data, 6, zdict=zdict)
    d = zlib.decompressobj(-15, zdict=zdict)
    assert d.decompress(stream) == data
    with no_cpu_codec:
        out = cuda_zlib.decompress_deflate_raw(stream, size, 0, zdict=zdict)
        assert out.cpu().numpy().tobytes() == data
        # Without the history the first back-reference has nothing to read.
        _, meta = cuda_zlib.decompress_deflate_raw_checked(stream, size, 0)
        assert _status(meta) == 6


def test_zlib_stream_without_fdict_ignores_a_dictionary(gpu, no_cpu_codec):
    import cuda_zlib
    data = _text(150000, 15)
    stream = zlib.compress(data, 6)
    with no_cpu_codec:
        out = cuda_zlib.decompress_zlib(stream, len(data), 0, zdict=b"unused dictionary")
    assert out.cpu().numpy().tobytes() == data


def test_format_entry_point_without_dictionary_matches_the_zlib_one(gpu):
    """Format 0 without a dictionary is HipZlibDecompress, statuses included."""
    import ctypes
    import torch
    import deflate_writer as dw
    from cuda_zlib import _native
    lib = _native.load()
    dev = torch.device("cuda", 0)
    for name, payload, expected, max_c, max_b, _, _ in dw.pinned_cases()[:40]:
        src = torch.frombuffer(bytearray(payload), dtype=torch.uint8).to(dev) if payload else \
            torch.empty(0, dtype=torch.uint8, device=dev)
        results = []
        for symbol in ("HipZlibDecompress", "HipZlibDecompressFormat"):
            out = torch.full((max(expected, 1),), 7, dtype=torch.uint8, device=dev)
            meta = torch.zeros(2, dtype=torch.uint32, device=dev)
            stream = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
            p = lambda t: ctypes.c_void_p(t.data_ptr() if t.numel() else 0)
            head = (stream,) if symbol == "HipZlibDecompress" else (stream, 0, None, 0)
            rc = getattr(lib, symbol)(*head, max_c, max_b, p(src), len(payload), p(out), expected,
                                      p(meta), 2)
            torch.cuda.synchronize(dev)
            results.append((rc, out[:expected].cpu().numpy().tobytes(), int(meta[0])))
        assert results[0] == results[1], name
