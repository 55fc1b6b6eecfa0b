"""Writes tests/golden/c0.json: the golden values of the 1 MiB text-like workload.

The workload (seed 0) is the plumbing case of the codec: 1 MiB of bytes drawn
from a 64-symbol alphabet (0x20-0x5F) with Zipf s=1.1 frequencies, then at
least 30 % overwritten by back-copies (length 8-64, distance 1-32768).  The
fixture records the SHA-256 of the raw bytes, their Adler-32, and the length
and SHA-256 of CPU zlib's level-6 stream of them, with the zlib version that
made it.  Run from the repository root: ``python tests/golden/make_golden.py``.
"""

import hashlib
import json
import os
import sys
import zlib

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

import workloads  # noqa: E402


def golden():
    raw = workloads.c0()
    stream = zlib.compress(raw, 6)
    return {
        "workload": "text-like, 1 MiB, seed 0 (Zipf 1.1 over 0x20-0x5F, >=30% back-copies)",
        "raw_len": len(raw),
        "raw_sha256": hashlib.sha256(raw).hexdigest(),
        "raw_head_hex": raw[:48].hex(),
        "adler32": zlib.adler32(raw),
        "zlib_version": zlib.ZLIB_RUNTIME_VERSION,
        "level6_len": len(stream),
        "level6_sha256": hashlib.sha256(stream).hexdigest(),
        "level1_len": len(zlib.compress(raw, 1)),
    }


if __name__ == "__main__":
    with open(os.path.join(HERE, "c0.json"), "w") as f:
        json.dump(golden(), f, indent=1)
        f.write("\n")
