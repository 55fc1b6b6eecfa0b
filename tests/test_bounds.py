"""CPU bounds checks of the device readers, built for the host with a guard page.

The readers, table builders and copies the kernels use (deflate_common.h:
BitIn, WordBits with fast_token, decode_token, the table builds, copy_bytes,
parse_frame) are compiled for the CPU (hipcc --offload-host-only, with
AddressSanitizer) by tests/bounds/guarded_readers.cpp, which places every
input so that it ends where a PROT_NONE page begins and decodes every
truncation of it.  Any read past a buffer is a crash here rather than a GPU
memory fault.  Valid streams must also decode completely to their size.
"""

import os
import shutil
import subprocess
import zlib

import numpy as np
import pytest

import deflate_writer as dw
import workloads
from conftest import ROOT

SOURCE = os.path.join(ROOT, "tests", "bounds", "guarded_readers.cpp")
HIPCC = os.path.join(os.environ.get("ROCM_PATH", "/opt/rocm"), "bin", "hipcc")


@pytest.fixture(scope="module")
def harness(tmp_path_factory):
    if not os.path.exists(HIPCC):
        pytest.skip("hipcc not available")
    out = str(tmp_path_factory.mktemp("bounds") / "guarded_readers")
    cmd = [HIPCC, "-x", "hip", "--offload-host-only", "-O1", "-g", "-std=c++17",
           "-fsanitize=address", "-I", os.path.join(ROOT, "cuda-zlib_amd", "csrc"), SOURCE,
           "-o", out]
    proc = subprocess.run(cmd, capture_output=True, text=True, timeout=600)
    assert proc.returncode == 0, proc.stderr[-3000:]
    return out


def _run(harness, mode, paths=()):
    proc = subprocess.run([harness, mode, *paths], capture_output=True, text=True, timeout=600)
    return proc


def _streams():
    """(name, zlib stream, decoded bytes or None) up to a few KB, so that every
    truncation of each is decoded."""
    rng = np.random.default_rng(17)
    text = workloads.text_like(3000, rng)
    noise = rng.integers(0, 256, 1200, dtype=np.uint8).tobytes()
    runs = b"a" * 700 + b"b" * 300 + bytes(range(50)) * 4
    out = []
    for name, raw in (("text", text), ("noise", noise), ("runs", runs), ("empty", b"")):
        for level in (0, 1, 6, 9):
            out.append(("%s-l%d" % (name, level), zlib.compress(raw, level), raw))
        for strategy, tag in ((zlib.Z_FIXED, "fixed"), (zlib.Z_RLE, "rle"),
                              (zlib.Z_HUFFMAN_ONLY, "huffman")):
            c = zlib.compressobj(6, zlib.DEFLATED, 15, 8, strategy)
            out.append(("%s-%s" % (name, tag), c.compress(raw) + c.flush(), raw))
    for name, payload, raw in dw.valid_streams():
        if len(payload) <= 6000:
            out.append(("valid-" + name, payload, raw))
    for case in dw.pinned_cases():
        if len(case[1]) <= 6000:
            out.append(("pinned-" + case[0], case[1], None))
    return out


@pytest.fixture(scope="module")
def stream_files(tmp_path_factory):
    d = tmp_path_factory.mktemp("streams")
    files = []
    for i, (name, payload, raw) in enumerate(_streams()):
        path = str(d / ("%03d.z" % i))
        with open(path, "wb") as f:
            f.write(payload)
        files.append((name, path, raw))
    return files


def _parse(stdout):
    result = {}
    for line in stdout.splitlines():
        fields = line.split()
        result[fields[0]] = dict(f.split("=") for f in fields[1:])
    return result


@pytest.mark.parametrize("mode", ["walk", "staged"])
def test_every_truncation_stays_inside_its_buffers(harness, stream_files, mode):
    proc = _run(harness, mode, [p for _, p, _ in stream_files])
    assert proc.returncode == 0, proc.stderr[-3000:]
    got = _parse(proc.stdout)
    assert len(got) == len(stream_files)
    for name, path, raw in stream_files:
        if raw is not None:
            assert got[path]["full"] == "0", name
            assert int(got[path]["bytes"]) == len(raw), name


def test_wrapper_parsing_of_every_truncation(harness, stream_files, tmp_path):
    gz = tmp_path / "member.gz"
    import gzip
    gz.write_bytes(gzip.compress(b"frame" * 50, 6, mtime=0))
    paths = [p for _, p, _ in stream_files[:12]] + [str(gz)]
    proc = _run(harness, "frame", paths)
    assert proc.returncode == 0, proc.stderr[-3000:]
    got = _parse(proc.stdout)
    assert got[str(gz)]["f2"] == "0" and got[str(gz)]["f0"] == "16"
    for p in paths[:-1]:
        assert got[p]["f0"] == "0" and got[p]["f1"] == "0" and got[p]["f2"] == "15"


def test_gzip_long_header_fields_every_truncation(harness, tmp_path):
    """A 3000-byte FNAME (terminated, with a comment and FHCRC; and one that
    runs into the trailer) parsed at every truncation from guarded buffers:
    no read past the end, and the full files give 0 and 14."""
    import struct
    name = bytes(range(1, 256)) * 12 + b"abcdefghijklmno"
    data = b"header fields " * 40
    header = bytes((0x1F, 0x8B, 8, 8 | 16 | 2)) + bytes(6) + name + b"\0" + b"comment\0"
    header += struct.pack("<H", zlib.crc32(header) & 0xFFFF)
    c = zlib.compressobj(6, zlib.DEFLATED, -15)
    good = header + c.compress(data) + c.flush() + struct.pack("<II", zlib.crc32(data), len(data))
    assert zlib.decompress(good, 31) == data
    runs_on = bytes((0x1F, 0x8B, 8, 8)) + bytes(6) + name + bytes(8)
    paths = []
    for label, blob in (("long_name.gz", good), ("runs_on.gz", runs_on)):
        path = tmp_path / label
        path.write_bytes(blob)
        paths.append(str(path))
    proc = _run(harness, "frame", paths)
    assert proc.returncode == 0, proc.stderr[-3000:]
    got = _parse(proc.stdout)
    assert got[paths[0]]["f2"] == "0" and got[paths[1]]["f2"] == "14"


def test_literal_pairs_match_single_tokens(harness, stream_files):
    """quick_pair (two literals per step) and quick_triple (three) stop at
    every slice end where quick_token does, end every step at one of its token
    starts and decode the same bytes: checked slice by slice in C, and the
    result against the bytes zlib produced."""
    valid = [(n, p, raw) for n, p, raw in stream_files if raw is not None]
    proc = _run(harness, "pairs", [p for _, p, _ in valid])
    assert proc.returncode == 0, proc.stderr[-3000:]
    got = _parse(proc.stdout)
    for name, path, raw in valid:
        for slice_bits in (29, 97, 512):
            assert got[path]["s%d" % slice_bits] == "0", (name, slice_bits)
            assert int(got[path]["bytes%d" % slice_bits]) == len(raw), name
            assert int(got[path]["adler%d" % slice_bits]) == zlib.adler32(raw), name


def test_window_token_matches_fast_token_at_every_bit(harness, stream_files):
    """The slow-path token decode from the window's registers (window_token)
    gives fast_token's status, token and end position at every bit of every
    block body, with the body end and with nearer limits as the bound."""
    proc = _run(harness, "window", [p for _, p, _ in stream_files])
    assert proc.returncode == 0, proc.stdout[-3000:] + proc.stderr[-2000:]
    lines = [l for l in proc.stdout.splitlines() if l.startswith("window ")]
    assert lines and all(l.endswith("bad=0") for l in lines)
    assert sum(int(l.split("positions=")[1].split()[0]) for l in lines) > 100000


def test_long_codes_match_a_bitwise_canonical_walk(harness):
    """Codes longer than the primary LUT are decoded from per-length bounds
    (deflate_common.h long_code); a bit-by-bit canonical walk must give the
    same symbol, length and error for every prefix the LUT misses, at every
    bit budget, on random complete (up to 15-bit), single-code and empty
    tables.  The wave build's per-lane bound formula is checked against the
    serial one on the same tables."""
    proc = _run(harness, "longcodes")
    assert proc.returncode == 0, proc.stdout[-3000:] + proc.stderr[-2000:]
    checked = int(proc.stdout.split("checked=")[1].split()[0])
    assert checked > 1000000 and "bad=0" in proc.stdout


def test_copy_bytes_every_length_and_alignment(harness):
    proc = _run(harness, "copy")
    assert proc.returncode == 0, proc.stdout + proc.stderr[-2000:]
    assert "copy cases=24832" in proc.stdout


def test_the_guard_page_catches_a_one_byte_overrun(harness):
    """The harness itself: a read of the first byte past a buffer must crash."""
    proc = _run(harness, "guard")
    assert proc.returncode != 0
    assert "SEGV" in proc.stderr or proc.returncode < 0
