#!/usr/bin/env python3
"""Benchmark of the MI355X zlib codec on the 64 MiB float32-strain stream.

One step = one decode of the 64 MiB (16,777,216 float32 samples) strain stream
compressed by CPU zlib level 6, with the compressed stream already resident in
HBM, through the codec's C ABI on the current stream.  Output is checked
bit-exact against the source after warmup and after the timed steps.

Prints one JSON line: value = uncompressed GB/s (wall clock between
synchronisations), a roofline entry for the dominant kernel (timed live with
HIP events on the codec's stream), the encoder on the same 64 MiB when
available, and CPU baselines measured on this host: the oracle's serial C
inflate (a port of the reference's serial decode), and zlib / libdeflate
single-thread and one process per core.
"""

import argparse
import ctypes
import ctypes.util
import json
import os
import statistics
import sys
import tempfile
import time
import zlib

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "cuda-zlib_amd"))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
MAX = 262144


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr() if t.numel() else 0)


# ---- CPU baselines ---------------------------------------------------------

def _zlib_worker(args):
    path, core, repeats, mode = args
    try:
        os.sched_setaffinity(0, {core})
    except OSError:
        pass
    with open(path, "rb") as f:
        payload = f.read()
    t0 = time.perf_counter()
    total = 0
    for _ in range(repeats):
        if mode == "decompress":
            total += len(zlib.decompress(payload))
        else:
            total += len(payload)
            zlib.compress(payload, 1)
    return total, time.perf_counter() - t0


def _all_cores(payload, mode, seconds_hint, single_rate, unit_bytes):
    """Aggregate throughput of one zlib process per core (at most 16 processes).

    single_rate is the single-thread rate in bytes/s; each process repeats the
    whole-stream operation enough times to run about seconds_hint seconds.
    """
    import multiprocessing as mp
    cores = sorted(os.sched_getaffinity(0))[:16]
    repeats = max(1, round(seconds_hint * single_rate / unit_bytes))
    with tempfile.NamedTemporaryFile(dir="/tmp", delete=False) as f:
        f.write(payload)
        path = f.name
    try:
        ctx = mp.get_context("spawn")
        with ctx.Pool(len(cores)) as pool:
            t0 = time.perf_counter()
            results = pool.map(_zlib_worker, [(path, c, repeats, mode) for c in cores])
            wall = time.perf_counter() - t0
        total = sum(r[0] for r in results)
        return total / wall / 1e9, len(cores), repeats
    finally:
        os.unlink(path)


def _libdeflate_decode(payload, size):
    name = ctypes.util.find_library("deflate")
    if not name:
        return None
    lib = ctypes.CDLL(name)
    lib.libdeflate_alloc_decompressor.restype = ctypes.c_void_p
    lib.libdeflate_zlib_decompress.argtypes = [ctypes.c_void_p, ctypes.c_char_p, ctypes.c_size_t,
                                               ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]
    d = lib.libdeflate_alloc_decompressor()
    out = ctypes.create_string_buffer(size)
    times = []
    for _ in range(3):
        t0 = time.perf_counter()
        rc = lib.libdeflate_zlib_decompress(d, payload, len(payload), out, size, None)
        times.append(time.perf_counter() - t0)
        if rc != 0:
            return None
    return size / statistics.median(times) / 1e9


def cpu_baselines(payload, raw, budget_s):
    from oracle import oracle
    n = len(raw)
    # Oracle port: the reference's serial decode restated in C, one core.
    t0 = time.perf_counter()
    out, status = oracle.inflate_serial(payload, n)
    port_s = time.perf_counter() - t0
    assert status == 0 and out == raw, "oracle failed on the benchmark stream"
    times = []
    for _ in range(3):
        t0 = time.perf_counter()
        zlib.decompress(payload)
        times.append(time.perf_counter() - t0)
    single = n / statistics.median(times) / 1e9
    all_cores, cores, repeats = _all_cores(payload, "decompress", budget_s, single * 1e9, n)
    t0 = time.perf_counter()
    zlib.compress(raw, 1)
    comp_single = n / (time.perf_counter() - t0) / 1e9
    comp_all, _, comp_repeats = _all_cores(raw, "compress", budget_s, comp_single * 1e9, n)
    return {
        "cpu_baseline": {"value": round(n / port_s / 1e9, 4), "unit": "GB/s", "cores": 1,
                         "kind": "port",
                         "sample": "full 64 MiB strain stream decoded once by the oracle's "
                                   "serial C inflate (restates the reference's serial decode)"},
        "cpu_zlib": {"zlib_version": zlib.ZLIB_RUNTIME_VERSION,
                     "decompress_single_gbs": round(single, 4),
                     "decompress_all_cores_gbs": round(all_cores, 4),
                     "compress_l1_single_gbs": round(comp_single, 4),
                     "compress_l1_all_cores_gbs": round(comp_all, 4),
                     "all_cores_processes": cores,
                     "repeats_per_process": {"decompress": repeats, "compress": comp_repeats},
                     "cpu_model": _cpu_model(),
                     "libdeflate_single_gbs": (lambda v: round(v, 4) if v else None)(
                         _libdeflate_decode(payload, n))},
    }


def _cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return None


# ---- GPU measurement ----------------------------------------------------------

def traffic_from_profiles(kernel):
    """HBM bytes per launch from the committed rocprofv3 PMC summary, if present."""
    path = os.path.join(ROOT, "profiles", "traffic.txt")
    if not os.path.exists(path):
        return None
    for line in open(path):
        parts = line.split()
        if len(parts) >= 2 and parts[0] == kernel:
            try:
                return int(float(parts[1]))
            except ValueError:
                return None
    return None


def main():
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=10)
    parser.add_argument("--warmup", type=int, default=2)
    parser.add_argument("--cpu-seconds", type=float, default=8.0,
                        help="approximate budget of each all-cores CPU baseline")
    parser.add_argument("--no-cpu-baseline", action="store_true")
    parser.add_argument("--legs", choices=("both", "decode", "encode"), default="both",
                        help="restrict the timed step to one leg (profiling runs)")
    parser.add_argument("--calibrate-copy", action="store_true",
                        help="run one plain 256 MiB device copy first, so that hardware "
                             "counters of a kernel with known traffic sit in the same profile")
    args = parser.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU: this codec path runs on a single MI355X; "
              "--gpus %d is not supported" % args.gpus, file=sys.stderr)
        return 2

    import numpy as np
    import torch
    import workloads
    from cuda_zlib import _native

    assert torch.cuda.is_available(), "bench.py needs a ROCm GPU"
    dev = torch.device("cuda", 0)
    lib = _native.load()
    raw = workloads.c1()
    payload = zlib.compress(raw, 6)
    n = len(raw)
    chunk = 32768
    chunks = (n + chunk - 1) // chunk
    capacity = n + 5 * chunks + 6
    src = torch.from_numpy(np.frombuffer(payload, np.uint8).copy()).to(dev)
    ref = torch.from_numpy(np.frombuffer(raw, np.uint8).copy()).to(dev)
    out = torch.empty(n, dtype=torch.uint8, device=dev)
    meta = torch.empty(2, dtype=torch.uint32, device=dev)
    enc = torch.empty(capacity, dtype=torch.uint8, device=dev)
    enc_meta = torch.empty(2, dtype=torch.uint32, device=dev)
    stream = torch.cuda.current_stream(dev)
    handle = ctypes.c_void_p(stream.cuda_stream)
    if args.calibrate_copy:
        a = torch.empty(256 << 20, dtype=torch.uint8, device=dev)
        b = torch.empty_like(a)
        torch.add(a, 1, out=b)  # elementwise kernel: reads and writes 256 MiB once
        torch.cuda.synchronize(dev)
        del a, b
    do_decode = args.legs in ("both", "decode")
    do_encode = args.legs in ("both", "encode")

    def decode():
        rc = lib.HipZlibDecompress(handle, MAX, MAX, _ptr(src), len(payload), _ptr(out), n,
                                   _ptr(meta), 2)
        if rc:
            _native.check(lib, rc)

    def encode():
        rc = lib.HipZlibCompress(handle, chunk, _ptr(ref), n, _ptr(enc), capacity,
                                 _ptr(enc_meta), 2)
        if rc:
            _native.check(lib, rc)

    def step():
        if do_decode:
            decode()
        if do_encode:
            encode()

    encoded = {}

    def verify(label):
        torch.cuda.synchronize(dev)
        if do_decode:
            status = int(meta.cpu().numpy()[0])
            assert status == 0, "%s: decode status %d" % (label, status)
            assert torch.equal(out, ref), "%s: decoded bytes differ from the source" % label
        if do_encode:
            length, status = (int(v) for v in enc_meta.cpu().numpy())
            assert status == 0, "%s: encode status %d" % (label, status)
            stream_bytes = enc[:length].cpu().numpy().tobytes()
            if "bytes" in encoded:
                assert stream_bytes == encoded["bytes"], "%s: encoder is not deterministic" % label
            else:
                assert zlib.decompress(stream_bytes) == raw, "%s: encoded stream fails zlib" % label
                encoded["bytes"] = stream_bytes

    for _ in range(max(1, args.warmup)):
        step()
    verify("warmup")
    out.zero_()
    enc.zero_()

    def timed(fn, steps):
        start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize(dev)
        t0 = time.perf_counter()
        start.record(stream)
        for _ in range(steps):
            fn()
        stop.record(stream)
        torch.cuda.synchronize(dev)
        return (time.perf_counter() - t0) * 1000 / steps, start.elapsed_time(stop) / steps

    ms_per_step, device_ms = timed(step, args.steps)
    verify("timed")
    value = n / (ms_per_step / 1000) / 1e9
    legs = {}
    if do_decode:
        legs["decode"] = timed(decode, max(3, args.steps // 2))
    if do_encode:
        legs["encode"] = timed(encode, max(3, args.steps // 2))

    # Per-kernel durations, HIP events around each launch on the codec's stream.
    lib.HipZlibProfileEnable(1)
    profile_steps = 3
    for _ in range(profile_steps):
        step()
    torch.cuda.synchronize(dev)
    lib.HipZlibProfileEnable(0)
    kernels = _native.profile_collect(lib)
    dominant, (launches, total_ms) = max(kernels.items(), key=lambda kv: kv[1][1])
    avg_ms = total_ms / launches
    # Algorithmic bytes per launch: the uncompressed bytes of the stream the
    # launch belongs to (one 64 MiB decode or encode per launch of every
    # per-step kernel).
    per_launch = n * profile_steps / launches
    achieved = per_launch / (avg_ms / 1000) / 1e9

    result = {
        "metric": "decompress+compress GB/s (uncompressed bytes), 64 MiB stream; % HBM peak",
        "value": round(value, 4),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "device_ms_per_step": round(device_ms, 4),
        "hbm_fraction": round(value / HBM_PEAK_GBS, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u8",
        "data": "synthetic (seeded float32 strain; decode input compressed by CPU zlib level 6)",
        "config": {"workload": "64 MiB float32 strain stream (16,777,216 samples, Gaussian sigma "
                               "1e-21 + 1e-22 chirp 20-500 Hz @ 4096 Hz, seed 1): one step = "
                               "decode of its zlib level-6 stream + encode with 32 KiB chunks"
                               if args.legs == "both" else
                               "64 MiB float32 strain stream, %s leg only" % args.legs,
                   "uncompressed_bytes": n, "compressed_bytes_l6": len(payload),
                   "chunk_bytes": chunk, "parallelism": "single GPU"},
        "legs": {k: {"gbs": round(n / (v[0] / 1000) / 1e9, 4), "ms": round(v[0], 4),
                     "device_ms": round(v[1], 4)} for k, v in legs.items()},
        "roofline": {"bound": "hbm", "kernel": dominant, "achieved": round(achieved, 3),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 6),
                     "traffic": traffic_from_profiles(dominant),
                     "avg_launch_ms": round(avg_ms, 4)},
        "kernels_ms_per_step": {k: round(v[1] / profile_steps, 4) for k, v in kernels.items()},
    }
    if "bytes" in encoded:
        result["encode_ratio"] = {"gpu": round(len(encoded["bytes"]) / n, 6),
                                  "zlib_l1": round(len(zlib.compress(raw, 1)) / n, 6),
                                  "zlib_l6": round(len(payload) / n, 6)}
    if not args.no_cpu_baseline:
        result.update(cpu_baselines(payload, raw, args.cpu_seconds))
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
