"""GPU decode parity: every route against the CPU oracle, through the C ABI."""

import random
import zlib

import pytest

import deflate_writer as dw
from gpu_helpers import capi_decompress
from oracle import oracle

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("case", dw.pinned_cases(), ids=lambda c: c[0])
def test_pinned_cases_match_oracle(gpu, case):
    name, payload, expected, max_candidates, max_blocks, status, output = case
    want, want_status = oracle.decompress(payload, expected, max_candidates, max_blocks)
    got, got_status, reserved = capi_decompress(payload, expected, max_candidates, max_blocks)
    assert reserved == 0
    assert got_status == want_status
    if status is not None:
        assert got_status == status
    assert got == want


@pytest.mark.parametrize("name,payload,raw", dw.valid_streams(), ids=lambda v: v if isinstance(v, str) else "")
@pytest.mark.parametrize("limits", ["default", "general"])
def test_valid_streams(gpu, name, payload, raw, limits):
    extra = () if limits == "default" else (4096, 65536)
    got, status, _ = capi_decompress(payload, len(raw), *extra)
    assert status == 0
    assert got == raw


def _corpus(seed, size):
    rng = random.Random(seed)
    kind = seed % 4
    if kind == 0:
        return bytes(rng.choices(b"the quick brown fox jumps over\n", k=size))
    if kind == 1:
        return rng.randbytes(size)
    if kind == 2:
        out = bytearray()
        while len(out) < size:
            out += bytes([rng.randrange(256)]) * rng.randint(1, 3000)
        return bytes(out[:size])
    words = [rng.randbytes(rng.randint(3, 12)) for _ in range(50)]
    return b"".join(rng.choice(words) for _ in range(size // 7))[:size]


@pytest.mark.parametrize("size", [70000, 300000, 2_000_000])
@pytest.mark.parametrize("level", [1, 6, 9])
@pytest.mark.parametrize("seed", range(4))
def test_general_route_zlib_streams(gpu, no_cpu_codec, size, level, seed):
    raw = _corpus(seed, size)
    payload = zlib.compress(raw, level)
    with no_cpu_codec:
        got, status, _ = capi_decompress(payload, len(raw))
    assert status == 0
    assert got == raw


@pytest.mark.parametrize("strategy", [zlib.Z_FILTERED, zlib.Z_HUFFMAN_ONLY, zlib.Z_RLE, zlib.Z_FIXED])
def test_general_route_strategies_and_flushes(gpu, strategy):
    raw = _corpus(3, 400000) + _corpus(2, 300000)
    c = zlib.compressobj(6, zlib.DEFLATED, 15, 8, strategy)
    parts = []
    for i in range(0, len(raw), 65536):
        parts.append(c.compress(raw[i:i + 65536]))
        parts.append(c.flush(zlib.Z_SYNC_FLUSH if i % 3 else zlib.Z_FULL_FLUSH))
    parts.append(c.flush())
    payload = b"".join(parts)
    got, status, _ = capi_decompress(payload, len(raw))
    assert status == 0 and got == raw


@pytest.mark.parametrize("seed", range(3))
def test_mutations_match_oracle(gpu, seed):
    rng = random.Random(100 + seed)
    raw = _corpus(seed, 90000)
    sources = [zlib.compress(raw, level) for level in (0, 1, 6)]
    for trial in range(40):
        src = bytearray(rng.choice(sources))
        for _ in range(rng.randint(1, 3)):
            i = rng.randrange(2, len(src))
            src[i] ^= 1 << rng.randrange(8)
        payload = bytes(src)
        expected = len(raw) + rng.choice([0, 0, 0, -1, 1])
        limits = rng.choice([(262144, 262144), (4096, 256)])
        want = oracle.decompress(payload, expected, *limits)
        got, status, _ = capi_decompress(payload, expected, *limits)
        assert (status, got) == (want[1], want[0]), "trial %d" % trial


def test_fast_chain_accepts_large_dynamic_blocks(gpu):
    """A strain stream (16 KiB dynamic blocks, ~120 kbit each) decodes through
    the parallel chain: the serial exact walk returns immediately."""
    import ctypes
    import numpy as np
    import torch
    import workloads
    from cuda_zlib import _native
    raw = workloads.strain((4 << 20) // 4, 1)
    payload = zlib.compress(raw, 6)
    lib = _native.load()
    dev = torch.device("cuda", 0)
    src = torch.from_numpy(np.frombuffer(payload, np.uint8).copy()).to(dev)
    out = torch.empty(len(raw), dtype=torch.uint8, device=dev)
    meta = torch.zeros(2, dtype=torch.uint32, device=dev)
    stream = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    _native.profile_collect(lib)
    lib.HipZlibProfileEnable(1)
    try:
        _native.check(lib, lib.HipZlibDecompress(stream, 262144, 262144, ctypes.c_void_p(src.data_ptr()),
                                                 len(payload), ctypes.c_void_p(out.data_ptr()),
                                                 len(raw), ctypes.c_void_p(meta.data_ptr()), 2))
        torch.cuda.synchronize(dev)
    finally:
        lib.HipZlibProfileEnable(0)
    kernels = _native.profile_collect(lib)
    assert int(meta.cpu().numpy()[0]) == 0
    assert out.cpu().numpy().tobytes() == raw
    assert kernels["g_exact_walk"][1] < 1.0, kernels["g_exact_walk"]
