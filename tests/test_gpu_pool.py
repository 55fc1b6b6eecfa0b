"""Workspace-pool controls on the GPU: retention, statistics, trimming, compile_kernels.

Follows the reference's pool interface (src/cuda_zlib/_ffi.py:175-184;
native/codec_ffi.cu:188-217, 1113-1142): the retention threshold can only be
set before the first pool exists, statistics report what the pool holds, and
a trim gives idle scratch back.  The retention checks run in a child process,
because the pool of this test process may already exist.
"""

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

CHILD = textwrap.dedent("""
    import ctypes, sys, zlib
    import numpy as np
    sys.path[:0] = [%(pkg)r, %(root)r]
    import cuda_zlib, workloads
    from cuda_zlib import _native
    lib = _native.load()
    print("step: stats before first use", flush=True)
    before = cuda_zlib.workspace_pool_stats(0)
    assert before["retention_bytes"] == %(retention)d, before
    assert before["pool_count"] == 0 and before["reserved_bytes"] == 0, before
    assert lib.HipZlibSetWorkspaceRetention(%(retention)d) == 0
    cuda_zlib.compile_kernels(0)
    raw = workloads.strain(1 << 19, 5)
    stream = zlib.compress(raw, 6)
    print("step: decode", flush=True)
    out = cuda_zlib.decompress_zlib(stream, len(raw), 0)
    assert out.cpu().numpy().tobytes() == raw
    after = cuda_zlib.workspace_pool_stats(0)
    assert after["pool_count"] == 1, after
    assert lib.HipZlibSetWorkspaceRetention(1) == _native.INVALID_ARGUMENT
    print("step: trim", flush=True)
    cuda_zlib.trim_workspace_pool(0)
    trimmed = cuda_zlib.workspace_pool_stats(0)
    print("stats", before, after, trimmed, flush=True)
    print("step: decode after trim", flush=True)
    again = cuda_zlib.decompress_zlib(stream, len(raw), 0)
    assert again.cpu().numpy().tobytes() == raw
    print("RESULT %%d %%d %%d" %% (after["reserved_bytes"], trimmed["reserved_bytes"],
                                  trimmed["used_bytes"]), flush=True)
""")


def _run_child(retention):
    env = dict(os.environ, CUDA_ZLIB_WORKSPACE_RETENTION_BYTES=str(retention))
    script = CHILD % {"pkg": os.path.join(ROOT, "cuda-zlib_amd"), "root": ROOT,
                      "retention": retention}
    proc = subprocess.run([sys.executable, "-c", script], env=env, capture_output=True,
                          text=True, timeout=300)
    print(proc.stdout)
    assert proc.returncode == 0, proc.stderr[-4000:]
    line = [l for l in proc.stdout.splitlines() if l.startswith("RESULT")][-1]
    return [int(v) for v in line.split()[1:]]


@pytest.mark.parametrize("retention", [256 << 20, 0], ids=["256MiB", "none"])
def test_retention_is_fixed_at_first_use_and_trim_releases_idle_scratch(gpu, retention):
    reserved, reserved_after_trim, used_after_trim = _run_child(retention)
    if retention:
        # The call's arena stays reserved until the trim gives it back.
        assert reserved > 0
        assert reserved_after_trim < reserved
    # An idle process: the trim frees the idle arenas and trims the pool empty.
    assert reserved_after_trim == 0
    assert used_after_trim == 0


def test_stats_and_trim_in_a_busy_process(gpu):
    import torch
    import cuda_zlib
    raw = workloads.text_like(3 << 20, np.random.default_rng(9))
    stream = zlib.compress(raw, 6)
    cuda_zlib.compile_kernels(0)
    out = cuda_zlib.decompress_zlib(stream, len(raw), 0)
    stats = cuda_zlib.workspace_pool_stats(torch.device("cuda", 0))
    assert stats["pool_count"] == 1
    assert set(stats) == {"retention_bytes", "reserved_bytes", "used_bytes", "pool_count"}
    # Work still queued when the trim runs keeps its scratch and finishes correctly.
    pending = cuda_zlib.decompress_zlib_checked(stream, len(raw), 0)
    cuda_zlib.trim_workspace_pool(0)
    torch.cuda.synchronize()
    assert int(pending[1][0]) == 0
    assert pending[0].cpu().numpy().tobytes() == raw == out.cpu().numpy().tobytes()
    cuda_zlib.trim_workspace_pool(0)
    assert cuda_zlib.workspace_pool_stats(0)["used_bytes"] == 0
