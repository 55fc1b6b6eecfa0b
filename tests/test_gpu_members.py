"""Concatenated zlib streams and multi-member gzip files (HIP_ZLIB_FORMAT_MEMBERS).

The reference refuses a second stream after the first
(tests/test_decode.py:679-713, case "concatenated"); the drop-in calls keep
that refusal (status 12).  With ``members=True`` every member decodes into one
output, which must equal what CPU zlib gives: ``gzip.decompress`` for gzip
files, and a ``zlib.decompressobj`` loop over ``unused_data`` for zlib
streams.  A failing member reports its own status.
"""

import gzip
import struct
import zlib

import numpy as np
import pytest

import workloads

pytestmark = pytest.mark.gpu

MIB = 1 << 20


def _payload(size, seed):
    """Alternating content: text-like and float32 strain bytes."""
    if seed % 2:
        return workloads.strain((size + 3) // 4, seed)[:size]
    return workloads.text_like(size, np.random.default_rng(seed))


def _gzip_file(parts, level=6):
    return b"".join(gzip.compress(p, level, mtime=0) for p in parts)


def _zlib_file(parts, level=6):
    return b"".join(zlib.compress(p, level) for p in parts)


def _zlib_loop(stream):
    """CPU zlib over a concatenation: one decompressobj per member, resumed on unused_data."""
    out = []
    while stream:
        d = zlib.decompressobj()
        out.append(d.decompress(stream))
        assert d.eof
        stream = d.unused_data
    return b"".join(out)


def _status(meta):
    return int(meta.cpu().numpy()[0])


def _sizes(count):
    cycle = [0, 100, 3 * MIB]
    return [cycle[i % 3] for i in range(count)]


@pytest.mark.parametrize("count", [1, 2, 17])
def test_gzip_members(gpu, no_cpu_codec, count):
    import cuda_zlib
    parts = [_payload(n, 40 + i) for i, n in enumerate(_sizes(count))]
    stream = _gzip_file(parts)
    want = gzip.decompress(stream)
    assert want == b"".join(parts)
    with no_cpu_codec:
        out, meta = cuda_zlib.decompress_gzip_checked(stream, len(want), 0, members=True)
        assert _status(meta) == 0
    assert out.cpu().numpy().tobytes() == want


@pytest.mark.parametrize("count", [1, 2, 17])
def test_zlib_members(gpu, no_cpu_codec, count):
    import cuda_zlib
    parts = [_payload(n, 60 + i) for i, n in enumerate(_sizes(count))]
    stream = _zlib_file(parts, level=1 + count % 9)
    want = _zlib_loop(stream)
    assert want == b"".join(parts)
    with no_cpu_codec:
        out = cuda_zlib.decompress_zlib(stream, len(want), 0, members=True)
    assert out.cpu().numpy().tobytes() == want


def test_member_larger_than_the_first_window(gpu, no_cpu_codec):
    """A member whose stream runs past the 16 MiB first look is decoded over the whole rest."""
    import cuda_zlib
    parts = [_payload(1000, 81), _payload(20 * MIB, 83), _payload(5000, 85)]
    stream = _gzip_file(parts, level=6)
    assert len(gzip.compress(parts[1], 6, mtime=0)) > 16 * MIB
    want = b"".join(parts)
    with no_cpu_codec:
        out = cuda_zlib.decompress_gzip(stream, len(want), 0, members=True)
    assert out.cpu().numpy().tobytes() == want


def test_single_member_matches_the_one_stream_call(gpu, no_cpu_codec):
    import cuda_zlib
    data = _payload(300000, 90)
    stream = zlib.compress(data, 6)
    with no_cpu_codec:
        a = cuda_zlib.decompress_zlib(stream, len(data), 0)
        b = cuda_zlib.decompress_zlib(stream, len(data), 0, members=True)
    assert a.cpu().numpy().tobytes() == b.cpu().numpy().tobytes() == data


def test_drop_in_calls_keep_refusing_a_second_stream(gpu, no_cpu_codec):
    import cuda_zlib
    parts = [_payload(70000, 91), _payload(70000, 92)]
    zlib_two, gzip_two = _zlib_file(parts), _gzip_file(parts)
    with no_cpu_codec:
        # The reference's case: the first stream's size, then bytes after it (12).
        _, meta = cuda_zlib.decompress_zlib_checked(zlib_two, 70000, 0)
        assert _status(meta) == 12
        _, meta = cuda_zlib.decompress_gzip_checked(gzip_two, 70000, 0)
        assert _status(meta) == 12
        # The size of both: the first stream ends short of it (11).
        _, meta = cuda_zlib.decompress_zlib_checked(zlib_two, 140000, 0)
        assert _status(meta) == 11


def _corrupt_trailer(member, xor):
    return member[:-8] + struct.pack("<I", struct.unpack("<I", member[-8:-4])[0] ^ xor) + \
        member[-4:]


def test_failing_second_member_reports_its_status(gpu, no_cpu_codec):
    import cuda_zlib
    parts = [_payload(200000, 93), _payload(3 * MIB, 94), _payload(100, 95)]
    members = [gzip.compress(p, 6, mtime=0) for p in parts]
    total = sum(len(p) for p in parts)
    cases = []
    # CRC-32 of member 2 wrong: 24, with the decoded bytes kept.
    cases.append(("crc", members[0] + _corrupt_trailer(members[1], 1) + members[2], 24, True))
    # Member 2's header damaged: 15, output cleared.
    bad = bytearray(members[1])
    bad[2] = 7
    cases.append(("header", members[0] + bytes(bad) + members[2], 15, False))
    # The input ends inside member 3's trailer: 14.
    cases.append(("trailer-cut", b"".join(members)[:-3], 14, False))
    # Bytes after the last member that start no member: 15.
    cases.append(("garbage-after", b"".join(members) + b"\x00" * 20, 15, False))
    for name, stream, status, keep in cases:
        with no_cpu_codec:
            out, meta = cuda_zlib.decompress_gzip_checked(stream, total, 0, members=True)
            got = _status(meta)
        assert got == status, name
        data = out.cpu().numpy().tobytes()
        if keep:
            assert data[:len(parts[0]) + len(parts[1])] == parts[0] + parts[1], name
        else:
            assert data == bytes(total), name
    # zlib: member 2's Adler-32 wrong gives 21.
    zm = [zlib.compress(p, 6) for p in parts]
    bad2 = zm[1][:-1] + bytes((zm[1][-1] ^ 1,))
    with no_cpu_codec:
        _, meta = cuda_zlib.decompress_zlib_checked(zm[0] + bad2 + zm[2], total, 0, members=True)
        assert _status(meta) == 21


def test_member_sizes_must_add_up(gpu, no_cpu_codec):
    import cuda_zlib
    parts = [_payload(80000, 96), _payload(1000, 97)]
    stream = _zlib_file(parts)
    total = sum(len(p) for p in parts)
    with no_cpu_codec:
        out, meta = cuda_zlib.decompress_zlib_checked(stream, total + 1, 0, members=True)
        assert _status(meta) == 11
        assert out.cpu().numpy().tobytes() == bytes(total + 1)
        _, meta = cuda_zlib.decompress_zlib_checked(stream, total - 1, 0, members=True)
        assert _status(meta) == 7


def test_members_of_empty_output(gpu, no_cpu_codec):
    import cuda_zlib
    stream = _gzip_file([b"", b"", b""])
    with no_cpu_codec:
        out, meta = cuda_zlib.decompress_gzip_checked(stream, 0, 0, members=True)
        assert _status(meta) == 0
    assert out.numel() == 0
