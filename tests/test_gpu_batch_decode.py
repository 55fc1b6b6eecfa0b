"""Batch decode parity: every file against the oracle's serial inflate.

Batch files of at least 32 B of output decode by parallel slices, one
workgroup per file; a file that does not decode cleanly there is handed to the
serial per-file decoder.  Either way each file's [status, 0] row and output
(decoded prefix then zeros on failure, the reference's DecodeOneFile,
native/batch_decode.cuh:123-296) must equal the oracle's serial inflate.
"""

import random
import zlib

import numpy as np
import pytest

import workloads
from oracle import oracle

pytestmark = pytest.mark.gpu


def _files(seed, count):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(count):
        size = int(rng.choice([0, 300, 1024, 5000, 40000, 70000, 150000]))
        kind = i % 3
        if kind == 0:
            raw = workloads.text_like(size, rng)
        elif kind == 1:
            raw = rng.normal(0.0, 1.0, (size + 3) // 4).astype("<f4").tobytes()[:size]
        else:
            raw = bytes(rng.integers(0, 256, size, dtype=np.uint8))
        level = int(rng.choice([1, 6, 9]))
        out.append((raw, zlib.compress(raw, level)))
    return out


def _mutate(payload, rng):
    data = bytearray(payload)
    kind = rng.randrange(5)
    if kind == 0 and len(data) > 8:  # flip a bit in the body
        i = rng.randrange(2, len(data) - 4)
        data[i] ^= 1 << rng.randrange(8)
    elif kind == 1 and len(data) > 12:  # truncate
        del data[rng.randrange(6, len(data) - 1):]
    elif kind == 2:  # wrong checksum
        data[-1] ^= 0x5A
    elif kind == 3 and len(data) > 8:  # overwrite a run of body bytes
        i = rng.randrange(2, len(data) - 4)
        for j in range(i, min(i + 16, len(data) - 4)):
            data[j] = rng.randrange(256)
    return bytes(data)


def _check(streams, expected):
    import torch
    from cuda_zlib import decompress_zlib_batch_checked
    out, meta = decompress_zlib_batch_checked(b"".join(streams), [len(s) for s in streams],
                                              expected, 0)
    torch.cuda.synchronize()
    host = out.cpu().numpy().tobytes()
    rows = meta.cpu().numpy()
    at = 0
    for i, (stream, n) in enumerate(zip(streams, expected)):
        want, want_status = oracle.inflate_serial(stream, n)
        assert int(rows[i, 1]) == 0
        assert int(rows[i, 0]) == want_status, "file %d: status %d, oracle %d" % (
            i, int(rows[i, 0]), want_status)
        assert host[at:at + n] == want, "file %d output differs" % i
        at += n


def test_valid_files_match_the_serial_oracle(gpu):
    files = _files(11, 48)
    _check([p for _, p in files], [len(r) for r, _ in files])


@pytest.mark.parametrize("seed", range(6))
def test_corrupted_files_match_the_serial_oracle(gpu, seed):
    rng = random.Random(seed)
    files = _files(100 + seed, 40)
    streams, expected = [], []
    for raw, payload in files:
        if rng.random() < 0.6:
            payload = _mutate(payload, rng)
        n = len(raw)
        if rng.random() < 0.1:
            n += rng.choice([-1, 1]) if n else 1
        streams.append(payload)
        expected.append(n)
    _check(streams, expected)


def test_codes_up_to_15_bits_on_both_batch_routes(gpu):
    """Files whose literal/length and distance codes run to 15 bits (most
    tokens miss the primary tables): large ones take the parallel route, the
    tiny ones the serial decoder; all must equal the oracle."""
    import deflate_writer as dw
    streams, expected = [], []
    for seed in range(6):
        payload, raw = dw.long_code_mix_stream(blocks=1 + seed % 3, tokens=[20, 400, 3000][seed % 3],
                                               seed=900 + seed)
        streams.append(payload)
        expected.append(len(raw))
    _check(streams, expected)


def test_stale_output_bytes_never_survive(gpu):
    """The batch decoders write every byte of every slot (the output is not
    cleared first): into an output buffer holding 0xA5 everywhere, valid,
    corrupted and size-mismatched files of both routes decode to the oracle's
    bytes (decoded prefix then zeros on failure), and the same buffer reused
    for a second batch keeps nothing of the first."""
    import ctypes
    import torch
    from cuda_zlib import _native
    from cuda_zlib._native import int64_array
    lib = _native.load()
    dev = torch.device("cuda", 0)
    stream = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    ptr = lambda t: ctypes.c_void_p(t.data_ptr())
    rng = random.Random(41)
    batches = []
    for seed in (300, 301):
        streams, expected = [], []
        for raw, payload in _files(seed, 36):
            if rng.random() < 0.5:
                payload = _mutate(payload, rng)
            n = len(raw)
            if rng.random() < 0.1:
                n += rng.choice([-1, 1]) if n else 1
            streams.append(payload)
            expected.append(n)
        batches.append((streams, expected))
    total = max(sum(e) for _, e in batches)
    out = torch.full((total,), 0xA5, dtype=torch.uint8, device=dev)
    for streams, expected in batches:
        payload = b"".join(streams)
        src = torch.from_numpy(np.frombuffer(payload, np.uint8).copy()).to(dev)
        n = sum(expected)
        meta = torch.empty((len(streams), 2), dtype=torch.uint32, device=dev)
        rc = lib.HipZlibDecompressBatch(stream, int64_array([len(s) for s in streams]),
                                        len(streams), int64_array(expected), len(expected),
                                        ptr(src), len(payload), ctypes.c_void_p(0), 0, 0,
                                        ptr(out), n, ptr(meta), len(streams), 2)
        assert rc == 0
        torch.cuda.synchronize()
        host = out[:n].cpu().numpy().tobytes()
        rows = meta.cpu().numpy()
        at = 0
        for i, (s, k) in enumerate(zip(streams, expected)):
            want, want_status = oracle.inflate_serial(s, k)
            assert int(rows[i, 0]) == want_status and int(rows[i, 1]) == 0, i
            assert host[at:at + k] == want, "file %d output differs" % i
            at += k


def test_encoded_rows_route_large_files_like_small_ones(gpu):
    """Bad [length, status] rows give 22 / 23 and zeroed outputs, large files too."""
    import torch
    from cuda_zlib import compress_zlib_batch_padded, decompress_zlib_batch_checked
    rng = np.random.default_rng(5)
    raws = [workloads.text_like(int(n), rng) for n in (200, 3000, 20000, 70000, 500, 9000)]
    sizes = [len(r) for r in raws]
    enc, meta = compress_zlib_batch_padded(b"".join(raws), sizes, 0)
    caps = [n + 5 * max(1, -(-n // 32768)) + 6 for n in sizes]
    rows = meta.clone()
    rows[1, 1] = 1            # a failed compression row
    rows[2, 0] = caps[2] + 1  # a stream longer than its slot
    rows[5, 1] = 22
    out, dmeta = decompress_zlib_batch_checked(enc, caps, sizes, 0, encoded_metadata=rows)
    torch.cuda.synchronize()
    status = dmeta.cpu().numpy()[:, 0].tolist()
    assert status == [0, 22, 23, 0, 0, 22]
    host = out.cpu().numpy().tobytes()
    at = 0
    for i, raw in enumerate(raws):
        got = host[at:at + len(raw)]
        assert got == (raw if status[i] == 0 else bytes(len(raw)))
        at += len(raw)


def _small_dynamic(rng, n):
    """A stream of under 256 B of output in one dynamic-Huffman block (most of
    them take the parallel route, those under 32 B the serial one)."""
    raw = bytes(rng.choice(b"abcdefg"[:rng.randrange(2, 8)]) for _ in range(n))
    c = zlib.compressobj(9, zlib.DEFLATED, 15, 9, zlib.Z_HUFFMAN_ONLY)
    return raw, c.compress(raw) + c.flush()


@pytest.mark.parametrize("seed", range(3))
def test_small_dynamic_headers_match_the_serial_oracle(gpu, seed):
    """Small files: under 32 B one wave per file, staged in LDS, their dynamic
    headers read by the wave walk (lane 0's serial parse where the walk
    stops), and above that by parallel slices with the serial decoder for
    any that fail; valid, header-corrupted and truncated ones against the
    oracle, beside large files so both routes run together."""
    rng = random.Random(40 + seed)
    streams, expected = [], []
    for i in range(60):
        raw, payload = _small_dynamic(rng, rng.randrange(1, 256))
        data = bytearray(payload)
        kind = rng.randrange(4)
        if kind == 1:  # a bit of the header fields, the code-length code or the lengths
            bit = rng.randrange(16 + 3, min(len(data) - 4, 40) * 8)
            data[bit // 8] ^= 1 << (bit % 8)
        elif kind == 2 and len(data) > 10:  # truncated inside the header
            del data[rng.randrange(3, min(len(data) - 1, 12)):]
        streams.append(bytes(data))
        expected.append(len(raw))
        if i % 10 == 0:  # a large neighbour for the parallel route
            big = workloads.text_like(rng.randrange(3000, 40000), np.random.default_rng(seed * 100 + i))
            streams.append(zlib.compress(big, 6))
            expected.append(len(big))
    _check(streams, expected)


def test_batch_on_a_side_stream_is_complete_when_that_stream_is(gpu):
    """A batch called on a non-default stream, with small and large files,
    is complete once that stream is synchronized."""
    import torch
    from cuda_zlib import decompress_zlib_batch_checked
    rng = random.Random(77)
    raws = []
    for i in range(200):
        if i % 4 == 0:
            raws.append(workloads.text_like(rng.randrange(2000, 60000), np.random.default_rng(i)))
        else:
            raws.append(_small_dynamic(rng, rng.randrange(1, 256))[0])
    streams = [zlib.compress(r, 6) for r in raws]
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        out, meta = decompress_zlib_batch_checked(b"".join(streams), [len(s) for s in streams],
                                                  [len(r) for r in raws], 0)
        host_out = torch.empty(out.numel(), dtype=torch.uint8, pin_memory=True)
        host_meta = torch.empty(meta.shape, dtype=meta.dtype, pin_memory=True)
        host_out.copy_(out, non_blocking=True)
        host_meta.copy_(meta, non_blocking=True)
    stream.synchronize()
    assert host_meta.numpy()[:, 0].tolist() == [0] * len(raws)
    assert host_out.numpy().tobytes() == b"".join(raws)


def test_batch_calls_on_two_streams_do_not_wait_for_each_other(gpu):
    """Batches on two caller streams are independent: a batch on stream B must
    finish while stream A, whose own batch waits behind a long kernel, is
    still busy."""
    import time
    import torch
    from cuda_zlib import decompress_zlib_batch_checked
    rng = random.Random(91)
    raws = []
    for i in range(64):
        if i % 4 == 0:
            raws.append(workloads.text_like(rng.randrange(2000, 20000), np.random.default_rng(i)))
        else:
            raws.append(_small_dynamic(rng, rng.randrange(1, 256))[0])
    packed = [zlib.compress(r, 6) for r in raws]
    payload = torch.from_numpy(np.frombuffer(b"".join(packed), np.uint8).copy()).cuda()
    sizes, expected = [len(s) for s in packed], [len(r) for r in raws]
    torch.cuda.synchronize()
    a, b = torch.cuda.Stream(), torch.cuda.Stream()
    with torch.cuda.stream(b):  # module, pools and side stream in place
        decompress_zlib_batch_checked(payload, sizes, expected, 0)
    b.synchronize()
    with torch.cuda.stream(a):
        torch.cuda._sleep(1 << 30)  # about half a second of spinning on stream A
        t0 = time.perf_counter()
        out_a, meta_a = decompress_zlib_batch_checked(payload, sizes, expected, 0)
        host_a = time.perf_counter() - t0
    if host_a > 0.1:
        pytest.skip("the call on the busy stream waited on the host (%.3f s)" % host_a)
    with torch.cuda.stream(b):
        out_b, meta_b = decompress_zlib_batch_checked(payload, sizes, expected, 0)
    b.synchronize()
    a_busy = not a.query()
    a.synchronize()
    assert a_busy, "stream B's batch finished only after stream A's work"
    for out, meta in ((out_a, meta_a), (out_b, meta_b)):
        assert meta.cpu().numpy()[:, 0].tolist() == [0] * len(raws)
        assert out.cpu().numpy().tobytes() == b"".join(raws)
