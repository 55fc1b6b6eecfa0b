"""HipZlibCompressNoAlloc: the compress entry point that allocates nothing.

Checked through the C ABI against HipZlibCompress on two calls in a row, the
second with a smaller input (the fixed scratch keeps the first call's
contents), plus CPU zlib round trips; an input whose scratch would not fit is
refused with a clear error; in a fresh process the entry point never creates
the scratch pool; one call captured in a HIP graph (torch.cuda.graph) and
replayed over inputs rewritten in place gives HipZlibCompress's streams.
"""

import ctypes
import os
import subprocess
import sys
import textwrap
import zlib

import numpy as np
import pytest

import workloads
from conftest import ROOT

pytestmark = pytest.mark.gpu


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr() if t.numel() else 0)


def _compress(lib, symbol, data, chunk):
    import torch
    dev = torch.device("cuda", 0)
    src = torch.frombuffer(bytearray(data), dtype=torch.uint8).to(dev) if data else \
        torch.empty(0, dtype=torch.uint8, device=dev)
    chunks = max(1, -(-len(data) // chunk))
    capacity = len(data) + 5 * chunks + 6
    out = torch.full((capacity,), 0xA5, dtype=torch.uint8, device=dev)
    meta = torch.full((2,), 0xDEAD, dtype=torch.uint32, device=dev)
    stream = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    rc = getattr(lib, symbol)(stream, chunk, _ptr(src), len(data), _ptr(out), capacity, _ptr(meta), 2)
    torch.cuda.synchronize(dev)
    return rc, out.cpu().numpy().tobytes(), [int(v) for v in meta.cpu().numpy()]


CALLS = [  # (input, chunk bytes): the second call is smaller than the first
    (lambda: workloads.text_like(9 << 20, np.random.default_rng(21)), 32768),
    (lambda: workloads.strain(70000, 22), 4096),
    (lambda: b"", 32768),
    (lambda: bytes(np.random.default_rng(23).integers(0, 256, 100000, dtype=np.uint8)), 65535),
]


def test_no_alloc_matches_the_allocating_entry_point_call_after_call(gpu):
    from cuda_zlib import _native
    lib = _native.load()
    for make, chunk in CALLS:
        data = make()
        rc_a, slot_a, meta_a = _compress(lib, "HipZlibCompress", data, chunk)
        rc_b, slot_b, meta_b = _compress(lib, "HipZlibCompressNoAlloc", data, chunk)
        assert rc_a == 0 and rc_b == 0
        assert meta_b == meta_a and meta_b[1] == 0
        assert slot_b == slot_a
        assert zlib.decompress(slot_b[:meta_b[0]]) == data


def test_no_alloc_refuses_an_input_whose_scratch_does_not_fit(gpu):
    from cuda_zlib import _native
    lib = _native.load()
    data = bytes(12 << 20)
    rc, slot, meta = _compress(lib, "HipZlibCompressNoAlloc", data, 32768)
    assert rc == _native.INVALID_ARGUMENT
    message = lib.HipZlibErrorString(rc).decode()
    assert "bytes of scratch" in message and "HipZlibCompress" in message
    assert meta == [0xDEAD, 0xDEAD] and set(slot[:4096]) == {0xA5}  # nothing was enqueued
    # Out-of-range chunk sizes get status 23 in the metadata, as HipZlibCompress gives.
    rc, _, meta = _compress(lib, "HipZlibCompressNoAlloc", b"abc", 100)
    assert rc == 0 and meta == [0, 23]


CHILD = textwrap.dedent("""
    import ctypes, sys, zlib
    sys.path[:0] = [%(pkg)r, %(root)r, %(tests)r]
    import torch
    import cuda_zlib, workloads
    from cuda_zlib import _native
    import test_zz_no_alloc as w
    lib = _native.load()
    data = workloads.strain(300000, 24)
    for chunk in (32768, 8192):
        rc, slot, meta = w._compress(lib, "HipZlibCompressNoAlloc", data, chunk)
        assert rc == 0 and meta[1] == 0, (rc, meta)
        assert zlib.decompress(slot[:meta[0]]) == data
    stats = cuda_zlib.workspace_pool_stats(0)
    assert stats["pool_count"] == 0, stats
    print("CHILD OK", flush=True)
""")


def test_fresh_process_never_creates_the_pool(gpu):
    script = CHILD % {"pkg": os.path.join(ROOT, "cuda-zlib_amd"), "root": ROOT,
                      "tests": os.path.join(ROOT, "tests")}
    proc = subprocess.run([sys.executable, "-c", script], capture_output=True, text=True,
                          timeout=300)
    assert proc.returncode == 0 and "CHILD OK" in proc.stdout, proc.stderr[-3000:]


def test_no_alloc_captured_in_a_graph_replays_over_new_inputs(gpu):
    """Capture one call, then replay it several times, the input rewritten in
    place between replays (eager work and a synchronisation around each), and
    check every replay against HipZlibCompress on the same bytes."""
    import torch
    from cuda_zlib import _native
    lib = _native.load()
    dev = torch.device("cuda", 0)
    n, chunk = 1 << 20, 32768
    capacity = n + 5 * (n // chunk) + 6
    inputs = [workloads.text_like(n, np.random.default_rng(31)), workloads.strain(n // 4, 32),
              bytes(np.random.default_rng(33).integers(0, 256, n, dtype=np.uint8))]
    src = torch.empty(n, dtype=torch.uint8, device=dev)
    out = torch.empty(capacity, dtype=torch.uint8, device=dev)
    meta = torch.empty(2, dtype=torch.uint32, device=dev)

    def call():
        stream = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
        return lib.HipZlibCompressNoAlloc(stream, chunk, _ptr(src), n, _ptr(out), capacity,
                                          _ptr(meta), 2)

    src.copy_(torch.frombuffer(bytearray(inputs[0]), dtype=torch.uint8))
    assert call() == 0  # eager first call: the device's scratch address is looked up here
    torch.cuda.synchronize(dev)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        rc = call()
    assert rc == 0
    for data in inputs + inputs[::-1]:
        host = torch.frombuffer(bytearray(data), dtype=torch.uint8)
        src.copy_(host)
        out.fill_(0xA5)
        meta.fill_(0xDEAD)
        torch.cuda.synchronize(dev)
        graph.replay()
        torch.cuda.synchronize(dev)
        length, status = (int(v) for v in meta.cpu().numpy())
        assert status == 0
        got = out.cpu().numpy().tobytes()
        assert zlib.decompress(got[:length]) == data
        rc, slot, meta_a = _compress(lib, "HipZlibCompress", data, chunk)
        assert rc == 0 and meta_a == [length, 0] and slot == got
