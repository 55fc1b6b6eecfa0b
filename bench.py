#!/usr/bin/env python3
"""Benchmark of the MI355X zlib codec on the 64 MiB float32-strain stream.

One step = one decode of the 64 MiB (16,777,216 float32 samples) strain stream
compressed by CPU zlib level 6, then one encode of the same 64 MiB with
32 KiB chunks, both on resident HBM buffers through the codec's C ABI on the
current stream.  Outputs are checked bit-exact after warmup and after the
timed steps.

Prints one JSON line on stdout: value = uncompressed GB/s of the round trip
(wall clock between synchronisations), each leg on its own, a roofline entry
for the dominant kernel (timed live with HIP events on the codec's stream),
the other workloads (256 MiB text encode, 4096-file batch, 1 GiB stress
stream decode, 64 MiB text decode, 16 MiB fixed-Huffman text decode, 64 KiB
text decode) timed the same way, and CPU baselines
measured on this host in the same run: Python zlib and libdeflate, one
thread and one pinned process per available core, and the oracle's serial C
inflate.  Progress lines go to stderr.
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

HBM_PEAK_GBS = 8000.0  # MI355X's published HBM3E bandwidth


def device_hbm_peak_gbs(device=0):
    """HBM peak from the device's own properties: memory clock (kHz) x bus
    width (bits) x 4 transfers a clock (HBM3E reports a quarter of its data
    rate: 2 GHz x 8192 bits x 4 = 8.19 TB/s on MI355X).  Recorded beside the
    published figure."""
    import ctypes
    hip = ctypes.CDLL("libamdhip64.so")
    bus, clock = ctypes.c_int(0), ctypes.c_int(0)
    # hipDeviceAttributeMemoryBusWidth = 59, hipDeviceAttributeMemoryClockRate = 60
    if hip.hipDeviceGetAttribute(ctypes.byref(bus), 59, device) or \
            hip.hipDeviceGetAttribute(ctypes.byref(clock), 60, device):
        return None
    return {"bus_bits": bus.value, "memory_clock_khz": clock.value,
            "peak_gbs": round(4.0 * clock.value * 1e3 * bus.value / 8 / 1e9, 1)}
MAX = 262144
SAMPLES = 5          # timed repetitions behind every median
MIB = 1 << 20


def log(message):
    print("[bench %.1fs] %s" % (time.perf_counter() - T0, message), file=sys.stderr, flush=True)


T0 = time.perf_counter()


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr() if t.numel() else 0)


# ---- CPU side: available cores, workers, libdeflate ---------------------------

def available_cpus():
    """Cores this process may run on: its affinity set, cut to the cgroup CPU quota.

    Returns (cores to use, description).  A quota below the affinity count means
    more processes than the quota would only share the same CPU time.
    """
    affinity = sorted(os.sched_getaffinity(0))
    quota = None
    try:
        fields = open("/sys/fs/cgroup/cpu.max").read().split()
        if fields and fields[0] != "max":
            quota = int(fields[0]) / int(fields[1])
    except (OSError, ValueError, IndexError):
        pass
    count = len(affinity) if quota is None else max(1, min(len(affinity), int(quota)))
    info = {"affinity_cpus": len(affinity), "cgroup_quota_cpus": quota,
            "host_cpus": os.cpu_count(), "processes": count, "cpu_model": _cpu_model()}
    return affinity[:count], info


def _cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return None


class LibDeflate:
    """ctypes binding of the system libdeflate (zlib-format calls), if present."""

    def __init__(self):
        name = ctypes.util.find_library("deflate")
        self.lib = ctypes.CDLL(name) if name else None
        if not self.lib:
            return
        p, sz = ctypes.c_void_p, ctypes.c_size_t
        self.lib.libdeflate_alloc_decompressor.restype = p
        self.lib.libdeflate_alloc_compressor.restype = p
        self.lib.libdeflate_alloc_compressor.argtypes = [ctypes.c_int]
        self.lib.libdeflate_zlib_decompress.argtypes = [p, ctypes.c_char_p, sz, p, sz, p]
        self.lib.libdeflate_zlib_compress.argtypes = [p, ctypes.c_char_p, sz, p, sz]
        self.lib.libdeflate_zlib_compress.restype = sz
        self.name = name

    def decompress(self, payload, size):
        d = self.lib.libdeflate_alloc_decompressor()
        out = ctypes.create_string_buffer(max(1, size))
        rc = self.lib.libdeflate_zlib_decompress(d, payload, len(payload), out, size, None)
        self.lib.libdeflate_free_decompressor(ctypes.c_void_p(d))
        if rc:
            raise RuntimeError("libdeflate decompress failed (%d)" % rc)
        return size

    def compress(self, data, level):
        c = self.lib.libdeflate_alloc_compressor(level)
        out = ctypes.create_string_buffer(len(data) + len(data) // 8 + 1024)
        n = self.lib.libdeflate_zlib_compress(c, data, len(data), out, len(out))
        self.lib.libdeflate_free_compressor(ctypes.c_void_p(c))
        if not n:
            raise RuntimeError("libdeflate compress failed")
        return n


def _operation(kind):
    """A callable (data) -> None for one CPU operation of the baseline set."""
    if kind == "zlib_decompress":
        return lambda data: zlib.decompress(data)
    if kind.startswith("zlib_compress"):
        level = int(kind[-1])
        return lambda data: zlib.compress(data, level)
    if kind.startswith("libdeflate"):
        ld = LibDeflate()
        if kind == "libdeflate_decompress":
            return lambda data: ld.decompress(data[1], data[0])
        level = int(kind[-1])
        return lambda data: ld.compress(data, level)
    if kind == "oracle_inflate":
        from oracle import oracle  # the oracle is the CPU baseline here, never the product
        return lambda data: oracle.inflate_serial(data[1], data[0])
    raise ValueError(kind)


def _load_input(path, kind):
    with open(path, "rb") as f:
        blob = f.read()
    if kind in ("libdeflate_decompress", "oracle_inflate"):
        size = int.from_bytes(blob[:8], "little")
        return (size, blob[8:])
    return blob


def _worker(args):
    """One pinned process: a warm-up call, then `repeats` timed calls after the barrier."""
    path, kind, core, repeats = args
    try:
        os.sched_setaffinity(0, {core})
    except OSError:
        pass
    data = _load_input(path, kind)
    op = _operation(kind)
    op(data)
    _BARRIER.wait()
    start = time.time()
    for _ in range(repeats):
        op(data)
    return start, time.time()


_BARRIER = None


def _init_worker(barrier):
    global _BARRIER
    _BARRIER = barrier


def _write_input(kind, data, size=None):
    f = tempfile.NamedTemporaryFile(dir="/tmp", delete=False, prefix="hzbench_")
    if kind in ("libdeflate_decompress", "oracle_inflate"):
        f.write(int(size).to_bytes(8, "little"))
    f.write(data)
    f.close()
    return f.name


def single_thread(kind, data, unit_bytes, size=None):
    """Median GB/s over SAMPLES calls (one warm-up) in this process."""
    payload = (size, data) if kind in ("libdeflate_decompress", "oracle_inflate") else data
    op = _operation(kind)
    op(payload)
    times = []
    for _ in range(SAMPLES):
        t0 = time.perf_counter()
        op(payload)
        times.append(time.perf_counter() - t0)
    return unit_bytes / statistics.median(times) / 1e9


def all_cores(kind, data, unit_bytes, cores, size=None):
    """Aggregate GB/s of one pinned process per core, each doing SAMPLES calls
    on its own copy, between a common start barrier and the last finish."""
    import multiprocessing as mp
    path = _write_input(kind, data, size)
    try:
        ctx = mp.get_context("spawn")
        barrier = ctx.Barrier(len(cores))
        with ctx.Pool(len(cores), initializer=_init_worker, initargs=(barrier,)) as pool:
            spans = pool.map(_worker, [(path, kind, c, SAMPLES) for c in cores], chunksize=1)
        wall = max(s[1] for s in spans) - min(s[0] for s in spans)
        return len(cores) * SAMPLES * unit_bytes / wall / 1e9
    finally:
        os.unlink(path)


def cpu_baselines(payload, raw, cores, cpu_info, text_sample):
    """CPU figures of the headline workload; returns the JSON keys to add."""
    n = len(raw)
    ld = LibDeflate()
    # Compression runs on a bounded sample (the first 8 MiB of the input) so
    # that every figure stays within a few seconds; decoding on the full stream.
    sample = raw[:8 * MIB]
    figures = {}

    def both(label, kind, data, unit, size=None):
        log("cpu baseline: %s" % label)
        figures[label + "_single_gbs"] = round(single_thread(kind, data, unit, size), 4)
        figures[label + "_all_cores_gbs"] = round(all_cores(kind, data, unit, cores, size), 4)

    both("zlib_decompress", "zlib_decompress", payload, n)
    both("zlib_compress_l1", "zlib_compress1", sample, len(sample))
    both("zlib_compress_l6", "zlib_compress6", sample, len(sample))
    if ld.lib:
        both("libdeflate_decompress", "libdeflate_decompress", payload, n, size=n)
        both("libdeflate_compress_l1", "libdeflate_compress1", sample, len(sample))
        both("libdeflate_compress_l6", "libdeflate_compress6", sample, len(sample))
    both("oracle_port_decompress", "oracle_inflate", payload, n, size=n)
    both("zlib_compress_l1_text", "zlib_compress1", text_sample, len(text_sample))

    def round_trip(dec, enc):
        return 1.0 / (1.0 / dec + 1.0 / enc)

    trip = round_trip(figures["zlib_decompress_all_cores_gbs"],
                      figures["zlib_compress_l1_all_cores_gbs"])
    return {
        "cpu_baseline": {
            "value": round(trip, 4), "unit": "GB/s", "cores": len(cores), "kind": "reference",
            "sample": "Python zlib %s (the reference's CPU path), one pinned process per "
                      "available core, each on its own copy: decode of the full 64 MiB strain "
                      "level-6 stream and level-1 compress of its first 8 MiB, %d calls each; "
                      "value = 1 / (1/decode + 1/compress), the round trip the headline times"
                      % (zlib.ZLIB_RUNTIME_VERSION, SAMPLES)},
        "cpu": dict(figures, zlib_version=zlib.ZLIB_RUNTIME_VERSION,
                    libdeflate=ld.name if ld.lib else None, samples=SAMPLES, **cpu_info),
    }


# ---- background generation of the other workloads ------------------------------

def _gen(task):
    """Runs in a worker process: builds one workload, writes it to /tmp files."""
    import numpy as np
    import workloads
    name = task
    out = {}
    t0 = time.perf_counter()
    if name == "c2":
        raw = workloads.c2()
        out["raw"] = _dump(raw)
        t = time.perf_counter()
        out["zlib_l1"] = len(zlib.compress(raw, 1))
        out["zlib_l1_s"] = time.perf_counter() - t
    elif name == "c2_l6":
        raw = workloads.c2()
        t = time.perf_counter()
        out["zlib_l6"] = len(zlib.compress(raw, 6))
        out["zlib_l6_s"] = time.perf_counter() - t
    elif name == "c4":
        payload, raw = workloads.c4()
        out["payload"], out["raw"] = _dump(payload), _dump(raw)
        t = time.perf_counter()
        zlib.decompress(payload)
        out["zlib_decompress_s"] = time.perf_counter() - t
    elif name == "text64":
        raw = workloads.text_like(64 * MIB, np.random.default_rng(5))
        payload = zlib.compress(raw, 6)
        out["payload"], out["raw"] = _dump(payload), _dump(raw)
        t = time.perf_counter()
        zlib.decompress(payload)
        out["zlib_decompress_s"] = time.perf_counter() - t
    elif name == "fixed16":
        raw = workloads.text_like(16 * MIB, np.random.default_rng(0))
        c = zlib.compressobj(1, zlib.DEFLATED, 15, 8, zlib.Z_FIXED)
        payload = c.compress(raw) + c.flush()
        out["payload"], out["raw"] = _dump(payload), _dump(raw)
        t = time.perf_counter()
        zlib.decompress(payload)
        out["zlib_decompress_s"] = time.perf_counter() - t
    elif name == "text64k":
        raw = workloads.text_like(64 * 1024, np.random.default_rng(7))
        payload = zlib.compress(raw, 6)
        out["payload"], out["raw"] = _dump(payload), _dump(raw)
        t = time.perf_counter()
        for _ in range(100):
            zlib.decompress(payload)
        out["zlib_decompress_s"] = (time.perf_counter() - t) / 100
    elif name == "c3":
        files = workloads.c3()
        out["files"] = _dump(b"".join(files))
        out["sizes"] = [len(f) for f in files]
        t = time.perf_counter()
        streams = [zlib.compress(f, 1) for f in files]
        out["zlib_l1_s"] = time.perf_counter() - t
        t = time.perf_counter()
        for s in streams:
            zlib.decompress(s)
        out["zlib_decompress_s"] = time.perf_counter() - t
    out["gen_s"] = time.perf_counter() - t0
    return name, out


def _dump(data):
    f = tempfile.NamedTemporaryFile(dir="/tmp", delete=False, prefix="hzbench_")
    f.write(data)
    f.close()
    return f.name


def _slurp(path):
    with open(path, "rb") as f:
        data = f.read()
    os.unlink(path)
    return data


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


class Gpu:
    def __init__(self, lib, native):
        import torch
        self.torch = torch
        self.dev = torch.device("cuda", 0)
        self.lib = lib
        self.native = native
        self.stream = torch.cuda.current_stream(self.dev)
        self.handle = ctypes.c_void_p(self.stream.cuda_stream)

    def tensor(self, data):
        import numpy as np
        return self.torch.from_numpy(np.frombuffer(data, np.uint8).copy()).to(self.dev)

    def empty(self, n, dtype=None):
        return self.torch.empty(n, dtype=dtype or self.torch.uint8, device=self.dev)

    def check(self, rc):
        if rc:
            self.native.check(self.lib, rc)

    def timed(self, fn, steps):
        """(wall ms, device ms) per call of `fn`, averaged over `steps` back-to-back calls."""
        torch = self.torch
        start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize(self.dev)
        t0 = time.perf_counter()
        start.record(self.stream)
        for _ in range(steps):
            fn()
        stop.record(self.stream)
        torch.cuda.synchronize(self.dev)
        return (time.perf_counter() - t0) * 1000 / steps, start.elapsed_time(stop) / steps

    def median_ms(self, fn, samples=SAMPLES):
        fn()
        runs = [self.timed(fn, 1)[0] for _ in range(samples)]
        return statistics.median(runs)

    def decode_call(self, src, n_in, out, n_out, meta):
        return lambda: self.check(self.lib.HipZlibDecompress(
            self.handle, MAX, MAX, _ptr(src), n_in, _ptr(out), n_out, _ptr(meta), 2))

    def encode_call(self, src, n, enc, capacity, meta, chunk=32768, independent=False):
        entry = self.lib.HipZlibCompressIndependent if independent else self.lib.HipZlibCompress
        return lambda: self.check(entry(
            self.handle, chunk, _ptr(src), n, _ptr(enc), capacity, _ptr(meta), 2))


def gbs(nbytes, ms):
    return round(nbytes / (ms / 1000) / 1e9, 4)


def extra_configs(gpu, generated):
    """Driver-timed figures of the other workloads; each checked bit-exact first."""
    import numpy as np
    result = {}
    torch = gpu.torch
    if "c2" in generated:
        info = generated["c2"]
        raw = _slurp(info["raw"])
        n = len(raw)
        chunks = (n + 32767) // 32768
        capacity = n + 5 * chunks + 6
        src, enc, meta = gpu.tensor(raw), gpu.empty(capacity), gpu.empty(2, torch.uint32)
        call = gpu.encode_call(src, n, enc, capacity, meta)
        log("c2: encode 256 MiB text")
        call()
        torch.cuda.synchronize()
        length, status = (int(v) for v in meta.cpu().numpy())
        assert status == 0, "c2 encode status %d" % status
        stream = enc[:length].cpu().numpy().tobytes()
        assert zlib.decompress(stream) == raw, "c2 stream fails zlib"
        ms = gpu.median_ms(call)
        # The same encode with every chunk's window confined to the chunk (the
        # reference's encoder semantics).
        call_ind = gpu.encode_call(src, n, enc, capacity, meta, independent=True)
        call_ind()
        torch.cuda.synchronize()
        length_ind, status = (int(v) for v in meta.cpu().numpy())
        assert status == 0, "c2 independent encode status %d" % status
        assert zlib.decompress(enc[:length_ind].cpu().numpy().tobytes()) == raw, \
            "c2 independent stream fails zlib"
        ms_ind = gpu.median_ms(call_ind)
        l6 = generated.get("c2_l6", {})
        result["c2_encode_256MiB_text"] = {
            "gbs": gbs(n, ms), "ms": round(ms, 3), "hbm_fraction": round(gbs(n, ms) / HBM_PEAK_GBS, 6),
            "ratio": round(length / n, 6), "zlib_l1_ratio": round(info["zlib_l1"] / n, 6),
            "zlib_l6_ratio": round(l6["zlib_l6"] / n, 6) if "zlib_l6" in l6 else None,
            "independent_chunks": {"gbs": gbs(n, ms_ind), "ms": round(ms_ind, 3),
                                   "ratio": round(length_ind / n, 6)},
            "cpu_zlib_l1_single_gbs": round(n / info["zlib_l1_s"] / 1e9, 4),
            "chunk_bytes": 32768, "round_trips_through": "zlib.decompress"}
        del src, enc, raw
    if "c3" in generated:
        info = generated["c3"]
        files = _slurp(info["files"])
        sizes = info["sizes"]
        total = len(files)
        caps = [s + 5 * max(1, (s + 32767) // 32768) + 6 for s in sizes]
        from cuda_zlib._native import int64_array
        src = gpu.tensor(files)
        slots, emeta = gpu.empty(sum(caps)), gpu.empty(len(sizes) * 2, torch.uint32)
        out, dmeta = gpu.empty(total), gpu.empty(len(sizes) * 2, torch.uint32)
        in_sizes, cap_sizes = int64_array(sizes), int64_array(caps)
        nfiles = len(sizes)

        def encode():
            gpu.check(gpu.lib.HipZlibCompressBatch(
                gpu.handle, 32768, in_sizes, nfiles, _ptr(src), total, _ptr(slots), sum(caps),
                _ptr(emeta), nfiles, 2))

        def decode():
            gpu.check(gpu.lib.HipZlibDecompressBatch(
                gpu.handle, cap_sizes, nfiles, in_sizes, nfiles, _ptr(slots), sum(caps),
                _ptr(emeta), nfiles, 2, _ptr(out), total, _ptr(dmeta), nfiles, 2))

        log("c3: batch of 4096 files")
        encode()
        decode()
        torch.cuda.synchronize()
        em = emeta.view(nfiles, 2).cpu().numpy()
        dm = dmeta.view(nfiles, 2).cpu().numpy()
        assert not em[:, 1].any() and not dm[:, 0].any(), "c3 statuses"
        assert torch.equal(out, src), "c3 batch round trip differs"
        enc_ms, dec_ms = gpu.median_ms(encode), gpu.median_ms(decode)
        result["c3_batch_4096_files"] = {
            "bytes": total, "encode_gbs": gbs(total, enc_ms), "encode_ms": round(enc_ms, 3),
            "decode_gbs": gbs(total, dec_ms), "decode_ms": round(dec_ms, 3),
            "ratio": round(float(em[:, 0].sum()) / total, 6),
            "cpu_zlib_l1_single_gbs": round(total / info["zlib_l1_s"] / 1e9, 4),
            "cpu_zlib_decompress_single_gbs": round(total / info["zlib_decompress_s"] / 1e9, 4)}
        del src, slots, out
    for key, label in (("c4", "c4_decode_1GiB_stress"), ("text64", "decode_64MiB_text_l6"),
                       ("fixed16", "decode_16MiB_text_fixed"), ("text64k", "decode_64KiB_text_l6")):
        if key not in generated:
            continue
        info = generated[key]
        payload, raw = _slurp(info["payload"]), _slurp(info["raw"])
        src, out, meta = gpu.tensor(payload), gpu.empty(len(raw)), gpu.empty(2, torch.uint32)
        ref = gpu.tensor(raw)
        del raw
        call = gpu.decode_call(src, len(payload), out, ref.numel(), meta)
        log("%s: decode" % key)
        call()
        torch.cuda.synchronize()
        assert int(meta[0]) == 0 and torch.equal(out, ref), "%s decode differs" % key
        ms = gpu.median_ms(call, 3 if key == "c4" else SAMPLES)
        n = ref.numel()
        result[label] = {"gbs": gbs(n, ms), "ms": round(ms, 3),
                         "hbm_fraction": round(gbs(n, ms) / HBM_PEAK_GBS, 6),
                         "compressed_bytes": len(payload),
                         "cpu_zlib_single_gbs": round(n / info["zlib_decompress_s"] / 1e9, 4)}
        if key == "text64k":
            # Device time of one decode: HIP events around 200 back-to-back calls.
            result[label]["device_us"] = round(gpu.timed(call, 200)[1] * 1000, 1)
            result[label]["cpu_zlib_single_us"] = round(info["zlib_decompress_s"] * 1e6, 1)
        del src, out, ref
    return result


def main():
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=10)
    parser.add_argument("--warmup", type=int, default=2)
    parser.add_argument("--no-cpu-baseline", action="store_true")
    parser.add_argument("--no-extra", action="store_true",
                        help="skip the other workloads (256 MiB text, batch, stress, text)")
    parser.add_argument("--legs", choices=("both", "decode", "encode"), default="both",
                        help="restrict the timed step to one leg (profiling runs; implies --no-extra)")
    parser.add_argument("--only", choices=("c2", "c3", "c4", "text64", "fixed16", "text64k"),
                        help="time one of the other workloads alone (profiling runs): prints "
                             "its figures as one JSON line, no headline")
    parser.add_argument("--calibrate-copy", action="store_true",
                        help="run one plain 256 MiB device copy first, so that hardware "
                             "counters of a kernel with known traffic sit in the same profile")
    args = parser.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU: this codec path runs on a single MI355X; "
              "--gpus %d is not supported" % args.gpus, file=sys.stderr)
        return 2
    extras = not args.no_extra and args.legs == "both"

    import multiprocessing as mp
    import numpy as np
    import torch
    import workloads
    from cuda_zlib import _native

    assert torch.cuda.is_available(), "bench.py needs a ROCm GPU"
    if args.only:
        lib = _native.load()
        gpu = Gpu(lib, _native)
        log("generating workload %s" % args.only)
        generated = dict([_gen(args.only)])
        if args.only == "c2":
            generated.update([_gen("c2_l6")])
        print(json.dumps({"workload": args.only, "configs": extra_configs(gpu, generated)}), flush=True)
        return 0
    cores, cpu_info = available_cpus()
    pool = pending = None
    if extras:
        # The other workloads are generated by CPU workers while the GPU runs
        # the headline; the CPU baselines run afterwards on idle cores.
        pool = mp.get_context("spawn").Pool(min(5, len(cores)))
        pending = pool.map_async(_gen, ["c2", "c2_l6", "c3", "c4", "text64", "fixed16", "text64k"])
    lib = _native.load()
    gpu = Gpu(lib, _native)
    log("generating the 64 MiB strain stream")
    raw = workloads.c1()
    payload = zlib.compress(raw, 6)
    n = len(raw)
    chunk = 32768
    chunks = (n + chunk - 1) // chunk
    capacity = n + 5 * chunks + 6
    src, ref = gpu.tensor(payload), gpu.tensor(raw)
    out, meta = gpu.empty(n), gpu.empty(2, torch.uint32)
    enc, enc_meta = gpu.empty(capacity), gpu.empty(2, torch.uint32)
    if args.calibrate_copy:
        a = gpu.empty(256 << 20)
        b = torch.empty_like(a)
        torch.add(a, 1, out=b)  # elementwise kernel: reads and writes 256 MiB once
        torch.cuda.synchronize(gpu.dev)
        del a, b
    do_decode = args.legs in ("both", "decode")
    do_encode = args.legs in ("both", "encode")
    decode = gpu.decode_call(src, len(payload), out, n, meta)
    encode = gpu.encode_call(ref, n, enc, capacity, enc_meta, chunk)

    def step():
        if do_decode:
            decode()
        if do_encode:
            encode()

    encoded = {}

    def verify(label):
        torch.cuda.synchronize(gpu.dev)
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

    log("warmup")
    for _ in range(max(1, args.warmup)):
        step()
    verify("warmup")
    out.zero_()
    enc.zero_()
    log("timed steps")
    ms_per_step, device_ms = gpu.timed(step, args.steps)
    verify("timed")
    value = n / (ms_per_step / 1000) / 1e9
    legs = {}
    if do_decode:
        legs["decode"] = gpu.timed(decode, max(3, args.steps // 2))
    if do_encode:
        legs["encode"] = gpu.timed(encode, max(3, args.steps // 2))

    # Per-kernel durations, HIP events around each launch on the codec's stream.
    lib.HipZlibProfileEnable(1)
    profile_steps = 3
    for _ in range(profile_steps):
        step()
    torch.cuda.synchronize(gpu.dev)
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
        "legs": {k: {"gbs": gbs(n, v[0]), "ms": round(v[0], 4), "device_ms": round(v[1], 4),
                     "hbm_fraction": round(gbs(n, v[0]) / HBM_PEAK_GBS, 6)}
                 for k, v in legs.items()},
        "roofline": {"bound": "hbm", "kernel": dominant, "achieved": round(achieved, 3),
                     "peak": HBM_PEAK_GBS, "peak_from_device": device_hbm_peak_gbs(),
                     "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 6),
                     "traffic": traffic_from_profiles(dominant),
                     "avg_launch_ms": round(avg_ms, 4)},
        "kernels_ms_per_step": {k: round(v[1] / profile_steps, 4) for k, v in kernels.items()},
        "launches_per_step": {k: round(v[0] / profile_steps, 2) for k, v in kernels.items()},
    }
    if "bytes" in encoded:
        result["encode_ratio"] = {"gpu": round(len(encoded["bytes"]) / n, 6),
                                  "zlib_l1": round(len(zlib.compress(raw, 1)) / n, 6),
                                  "zlib_l6": round(len(payload) / n, 6)}
    del src, out, enc
    if pending is not None:
        log("waiting for the other workloads")
        generated = dict(pending.get(timeout=900))
        pool.close()
        pool.join()
        result["configs"] = extra_configs(gpu, generated)
    if not args.no_cpu_baseline:
        text_sample = workloads.text_like(8 * MIB, np.random.default_rng(2))
        result.update(cpu_baselines(payload, raw, cores, cpu_info, text_sample))
        cpu = result["cpu"]
        result["gpu_vs_cpu_all_cores"] = {
            "round_trip": round(value / result["cpu_baseline"]["value"], 3),
            "decode_vs_zlib": round(result["legs"]["decode"]["gbs"] / cpu["zlib_decompress_all_cores_gbs"], 3)
            if "decode" in result["legs"] else None,
            "decode_vs_libdeflate": round(result["legs"]["decode"]["gbs"] /
                                          cpu["libdeflate_decompress_all_cores_gbs"], 3)
            if "decode" in result["legs"] and "libdeflate_decompress_all_cores_gbs" in cpu else None,
            "encode_vs_zlib_l1": round(result["legs"]["encode"]["gbs"] / cpu["zlib_compress_l1_all_cores_gbs"], 3)
            if "encode" in result["legs"] else None,
        }
    log("done")
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
