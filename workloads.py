"""Seeded synthetic workloads of the benchmark configurations (C0-C4).

Every generator uses ``numpy.random.default_rng(seed)`` and returns bytes, so
each workload is reproducible bit for bit; tests pin their SHA-256 digests.

C0  1 MiB text-like bytes (seed 0), zlib level 6: golden CPU round trip.
C1  64 MiB float32 "strain" (seed 1): Gaussian noise sigma 1e-21 plus a
    1e-22 chirp sweeping 20->500 Hz at 4096 Hz, zlib level 6: GPU decode.
C2  256 MiB text-like bytes (seed 2): GPU encode, chunk_bytes 32768.
C3  4096 small files (seed 3), log-uniform sizes in [16 B, 64 KiB], 64 empty,
    content cycling text / float32 noise / uniform random: batch encode+decode.
C4  1 GiB stress stream (seed 4): 1 MiB segments cycling stored (level 0),
    fixed Huffman (level 1, Z_FIXED), run-length (Z_RLE) and strain (level 9),
    one zlib stream with sync flushes: GPU decode.
"""

import zlib

import numpy as np

MIB = 1 << 20


def text_like(n, rng):
    """Zipf(s=1.1) bytes over 0x20..0x5F, then ~30% overwritten by back-copies.

    Copies have length U{8..64} and distance U{1..min(32768, n-L)}, land at
    U{d..n-L} and are applied forward byte by byte (an overlapping copy repeats
    its seed).  Copying stops once the copied byte count reaches 30% of n.
    """
    if n == 0:
        return b""
    ranks = np.arange(1, 65, dtype=np.float64)
    p = ranks ** -1.1
    p /= p.sum()
    data = (rng.choice(64, size=n, p=p) + 0x20).astype(np.uint8)
    target = int(0.3 * n)
    copied = attempts = 0
    # Parameters are drawn in batches and applied in order (a later copy may
    # read an earlier one).  Distances are capped at n - length so small files
    # still receive copies; for n >= 32832 the cap never binds.
    while copied < target and attempts < 4 * n + 64:
        batch = 4096
        lengths = rng.integers(8, 65, size=batch)
        u_dist = rng.random(batch)
        u_pos = rng.random(batch)
        for length, ud, up in zip(lengths.tolist(), u_dist.tolist(), u_pos.tolist()):
            attempts += 1
            if copied >= target:
                break
            dmax = min(32768, n - length)
            if dmax < 1:
                continue
            dist = 1 + int(ud * dmax)
            pos = dist + int(up * (n - length - dist + 1))
            src = pos - dist
            if dist >= length:
                data[pos:pos + length] = data[src:src + length]
            else:
                data[pos:pos + length] = np.resize(data[src:pos], length)
            copied += length
    return data.tobytes()


def c0():
    return text_like(MIB, np.random.default_rng(0))


def strain(samples, seed):
    rng = np.random.default_rng(seed)
    fs, f0, f1 = 4096.0, 20.0, 500.0
    t = np.arange(samples, dtype=np.float64) / fs
    duration = (samples - 1) / fs if samples > 1 else 1.0
    phase = 2 * np.pi * (f0 * t + (f1 - f0) * t * t / (2 * duration))
    x = rng.normal(0.0, 1e-21, samples) + 1e-22 * np.sin(phase)
    return x.astype("<f4").tobytes()


def c1():
    return strain(16 * MIB, 1)


def c2(size=256 * MIB):
    return text_like(size, np.random.default_rng(2))


def c3():
    rng = np.random.default_rng(3)
    n = 4096
    sizes = np.floor(np.exp(rng.uniform(np.log(16), np.log(65536), n))).astype(np.int64)
    sizes[rng.choice(n, 64, replace=False)] = 0
    files = []
    for i, size in enumerate(sizes.tolist()):
        kind = i % 3
        if kind == 0:
            files.append(text_like(size, rng))
        elif kind == 1:
            words = (size + 3) // 4
            files.append(rng.normal(0.0, 1.0, words).astype("<f4").tobytes()[:size])
        else:
            files.append(rng.integers(0, 256, size, dtype=np.uint8).tobytes())
    return files


def runs_segment(n, rng):
    out = bytearray()
    while len(out) < n:
        out += bytes([int(rng.integers(0, 256))]) * int(rng.integers(1, 100001))
    return bytes(out[:n])


def c4(segments=1024, segment=MIB):
    """Returns (payload, raw) of the mixed stress stream."""
    rng = np.random.default_rng(4)
    methods = [(0, zlib.Z_DEFAULT_STRATEGY), (1, zlib.Z_FIXED), (6, zlib.Z_RLE),
               (9, zlib.Z_DEFAULT_STRATEGY)]
    parts, raws = [b"\x78\x9c"], []
    adler = zlib.adler32(b"")
    history = b""
    for i in range(segments):
        kind = i % 4
        if kind == 0:
            raw = rng.integers(0, 256, segment, dtype=np.uint8).tobytes()
        elif kind == 1:
            raw = text_like(segment, rng)
        elif kind == 2:
            raw = runs_segment(segment, rng)
        else:
            raw = strain(segment // 4, int(rng.integers(1 << 31)))
        level, strategy = methods[kind]
        kwargs = {"zdict": history} if history else {}
        c = zlib.compressobj(level, zlib.DEFLATED, -15, 8, strategy, **kwargs)
        last = i == segments - 1
        parts.append(c.compress(raw) + c.flush(zlib.Z_FINISH if last else zlib.Z_SYNC_FLUSH))
        adler = zlib.adler32(raw, adler)
        history = (history + raw)[-32768:]
        raws.append(raw)
    parts.append(adler.to_bytes(4, "big"))
    return b"".join(parts), b"".join(raws)
