"""GPU encoder: every stream round-trips through CPU zlib, ratio bars, batch parity.

The encoder's contract (the reference's compress path, native/codec_ffi.cu:551-612
and src/cuda_zlib/_codec.py:142-205) is a valid zlib stream of at most
``n + 5 * chunks + 6`` bytes with metadata ``[encoded_length, status]``;
streams are checked with CPU ``zlib.decompress`` and the oracle's decoder.
"""

import ctypes
import zlib

import numpy as np
import pytest

import workloads
from gpu_helpers import _ptr, _tensor, capi_decompress
from oracle import oracle

pytestmark = pytest.mark.gpu


def _compress(data, chunk=32768):
    from cuda_zlib import compress_zlib_padded
    out, meta = compress_zlib_padded(data, 0, chunk_bytes=chunk)
    length, status = (int(v) for v in meta.cpu().numpy())
    assert status == 0
    chunks = max(1, -(-len(data) // chunk))
    assert out.numel() == len(data) + 5 * chunks + 6
    host = out.cpu().numpy().tobytes()
    assert not any(host[length:]), "padding after the stream must be zero"
    return host[:length]


def _kinds(n, seed):
    rng = np.random.default_rng(seed)
    yield "text", workloads.text_like(n, rng)
    yield "random", rng.integers(0, 256, n, dtype=np.uint8).tobytes()
    yield "zeros", bytes(n)
    yield "strain", workloads.strain(n // 4 + 1, seed)[:n]
    yield "period3", (b"abc" * (n // 3 + 1))[:n]


def test_empty_stream_bytes(gpu):
    stream = _compress(b"")
    assert stream == bytes.fromhex("7801030000000001")
    assert zlib.decompress(stream) == b""


@pytest.mark.parametrize("n", [1, 2, 3, 4, 255, 256, 257, 4095, 32767, 32768, 32769, 100003])
def test_round_trip_sizes(gpu, n):
    for kind, data in _kinds(n, n):
        stream = _compress(data)
        assert zlib.decompress(stream) == data, kind
        assert stream[:2] == b"\x78\x01"
        assert int.from_bytes(stream[-4:], "big") == zlib.adler32(data), kind


# 35000-byte chunks still parse two workgroups per CU (with less than 9 KiB
# of history), 36864-byte chunks take a whole CU.
@pytest.mark.parametrize("chunk", [256, 1000, 4096, 32768, 35000, 36864, 65535])
def test_round_trip_chunk_sizes(gpu, chunk):
    for kind, data in _kinds(300_001, chunk):
        stream = _compress(data, chunk)
        assert zlib.decompress(stream) == data, kind


def test_stream_decodes_in_the_oracle_and_on_the_gpu(gpu):
    data = workloads.text_like(700_000, np.random.default_rng(7))
    stream = _compress(data)
    out, status = oracle.decompress(stream, len(data))
    assert status == 0 and out == data
    got, status, _ = capi_decompress(stream, len(data))
    assert status == 0 and got == data


def test_ratio_c0_within_two_percent_of_zlib_level1(gpu):
    data = workloads.c0()
    stream = _compress(data)
    assert zlib.decompress(stream) == data
    ours, level1 = len(stream), len(zlib.compress(data, 1))
    assert ours <= 1.02 * level1, (ours, level1)


def test_ratio_text_16mib_within_two_percent_of_zlib_level1(gpu):
    data = workloads.text_like(16 << 20, np.random.default_rng(2))
    stream = _compress(data)
    assert zlib.decompress(stream) == data
    ours, level1 = len(stream), len(zlib.compress(data, 1))
    assert ours <= 1.02 * level1, (ours, level1)


def test_ratio_strain_within_two_percent_of_zlib_level1(gpu):
    data = workloads.strain(1 << 20, 1)
    stream = _compress(data)
    assert zlib.decompress(stream) == data
    ours, level1 = len(stream), len(zlib.compress(data, 1))
    assert ours <= 1.02 * level1, (ours, level1)


def test_incompressible_uses_stored_blocks_at_the_bound(gpu):
    data = np.random.default_rng(5).integers(0, 256, 100_000, dtype=np.uint8).tobytes()
    stream = _compress(data)
    assert zlib.decompress(stream) == data
    chunks = -(-len(data) // 32768)
    assert len(stream) == len(data) + 5 * chunks + 6


def _compress_independent(data, chunk=32768):
    from cuda_zlib import compress_zlib_padded
    out, meta = compress_zlib_padded(data, 0, chunk_bytes=chunk, independent_chunks=True)
    length, status = (int(v) for v in meta.cpu().numpy())
    assert status == 0
    host = out.cpu().numpy().tobytes()
    assert not any(host[length:]), "padding after the stream must be zero"
    return host[:length]


@pytest.mark.parametrize("chunk", [256, 4096, 32768])
def test_independent_chunks_round_trip(gpu, chunk):
    for kind, data in _kinds(200_003, chunk + 1):
        stream = _compress_independent(data, chunk)
        assert zlib.decompress(stream) == data, kind


@pytest.mark.parametrize("chunk", [8192, 16384])
def test_independent_chunks_never_reach_into_the_previous_chunk(gpu, chunk):
    """Two copies of an incompressible chunk: with history the second chunk is
    matches into the first (chunks up to 16 KiB keep at least a chunk of
    history); without history both chunks must be stored."""
    x = np.random.default_rng(21).integers(0, 256, chunk, dtype=np.uint8).tobytes()
    data = x + x
    shared = _compress(data, chunk)
    alone = _compress_independent(data, chunk)
    assert zlib.decompress(shared) == data and zlib.decompress(alone) == data
    assert len(shared) < chunk + chunk // 8
    assert len(alone) == len(data) + 5 * 2 + 6  # two stored chunks at the bound


def test_independent_chunks_cost_ratio_on_text(gpu):
    data = workloads.text_like(2 << 20, np.random.default_rng(23))
    shared, alone = _compress(data), _compress_independent(data)
    assert zlib.decompress(alone) == data
    assert len(shared) < len(alone) < len(data)


def test_deterministic(gpu):
    data = workloads.text_like(200_000, np.random.default_rng(11))
    assert _compress(data) == _compress(data)


def test_metadata_contract_and_bounds_through_the_c_abi(gpu):
    import torch
    from cuda_zlib import _native
    lib = _native.load()
    dev = torch.device("cuda", 0)
    data = b"hello hello hello hello"
    inp = _tensor(data, dev)
    stream = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    cap = len(data) + 5 + 6
    out = torch.full((cap,), 0xAB, dtype=torch.uint8, device=dev)
    meta = torch.full((2,), 0xDEAD, dtype=torch.uint32, device=dev)
    _native.check(lib, lib.HipZlibCompress(stream, 32768, _ptr(inp), len(data), _ptr(out), cap,
                                           _ptr(meta), 2))
    length, status = (int(v) for v in meta.cpu().numpy())
    assert status == 0
    assert zlib.decompress(out.cpu().numpy().tobytes()[:length]) == data
    # Wrong capacity and chunk size out of range: zeroed output, status 23.
    for chunk, size in ((32768, cap - 1), (255, cap), (65536, cap)):
        out = torch.full((size,), 0xAB, dtype=torch.uint8, device=dev)
        _native.check(lib, lib.HipZlibCompress(stream, chunk, _ptr(inp), len(data), _ptr(out),
                                               size, _ptr(meta), 2))
        assert [int(v) for v in meta.cpu().numpy()] == [0, 23]
        assert not out.cpu().numpy().any()


def _batch_files(seed, count):
    rng = np.random.default_rng(seed)
    files = []
    for i in range(count):
        size = int(np.exp(rng.uniform(np.log(16), np.log(200_000)))) if i % 7 else 0
        kind = i % 3
        if kind == 0:
            files.append(workloads.text_like(size, rng))
        elif kind == 1:
            files.append(rng.normal(0, 1, size // 4 + 1).astype("<f4").tobytes()[:size])
        else:
            files.append(rng.integers(0, 256, size, dtype=np.uint8).tobytes())
    return files


@pytest.mark.parametrize("chunk", [32768, 4096])
def test_batch_matches_single_streams(gpu, chunk):
    from cuda_zlib import compress_zlib_batch_padded
    files = _batch_files(3, 40)
    sizes = tuple(len(f) for f in files)
    out, meta = compress_zlib_batch_padded(b"".join(files), sizes, 0, chunk_bytes=chunk)
    meta = meta.cpu().numpy()
    host = out.cpu().numpy().tobytes()
    offset = 0
    for i, data in enumerate(files):
        chunks = max(1, -(-len(data) // chunk))
        cap = len(data) + 5 * chunks + 6
        length, status = int(meta[i, 0]), int(meta[i, 1])
        assert status == 0
        stream = host[offset:offset + length]
        assert not any(host[offset + length:offset + cap])
        assert zlib.decompress(stream) == data
        assert stream == _compress(data, chunk), "batch stream differs from single stream %d" % i
        offset += cap


def test_batch_round_trip_through_padded_slots(gpu):
    from cuda_zlib import compress_zlib_batch_padded, decompress_zlib_batch_checked
    files = _batch_files(4, 64)
    sizes = tuple(len(f) for f in files)
    out, meta = compress_zlib_batch_padded(b"".join(files), sizes, 0)
    caps = tuple(n + 5 * max(1, -(-n // 32768)) + 6 for n in sizes)
    decoded, dmeta = decompress_zlib_batch_checked(out, caps, sizes, 0, encoded_metadata=meta)
    dmeta = dmeta.cpu().numpy()
    assert not dmeta.any()
    assert decoded.cpu().numpy().tobytes() == b"".join(files)


def test_public_api_round_trip(gpu, no_cpu_codec):
    from cuda_zlib import (compress_zlib, compress_zlib_batch, compress_zlib_batch_host,
                           decompress_zlib, decompress_zlib_batch)
    data = workloads.text_like(123_457, np.random.default_rng(9))
    files = [data[:1000], b"", data[1000:50_000]]
    with no_cpu_codec:
        stream = compress_zlib(data)
        back = decompress_zlib(stream, len(data))
        streams = compress_zlib_batch(files)
        host_streams = compress_zlib_batch_host(files)
        backs = decompress_zlib_batch(streams, [len(f) for f in files])
    assert back.cpu().numpy().tobytes() == data
    assert zlib.decompress(stream.cpu().numpy().tobytes()) == data
    assert [b.cpu().numpy().tobytes() for b in backs] == files
    assert [zlib.decompress(s) for s in host_streams] == files
