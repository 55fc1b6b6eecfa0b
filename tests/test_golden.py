"""The 1 MiB text-like workload against its committed golden values.

tests/golden/c0.json (written by tests/golden/make_golden.py) holds the SHA-256
of the raw bytes, their Adler-32 and CPU zlib's level-6 stream.  The CPU tests
pin the generator and the oracle on it; the GPU tests decode the golden stream
and encode the raw bytes through the C ABI.
"""

import hashlib
import json
import os
import zlib

import pytest

import workloads
from oracle import oracle

GOLDEN = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "c0.json")))


@pytest.fixture(scope="module")
def c0():
    raw = workloads.c0()
    return raw, zlib.compress(raw, 6)


def test_generator_matches_golden(c0):
    raw, stream = c0
    assert len(raw) == GOLDEN["raw_len"]
    assert raw[:48].hex() == GOLDEN["raw_head_hex"]
    assert hashlib.sha256(raw).hexdigest() == GOLDEN["raw_sha256"]
    assert zlib.adler32(raw) == GOLDEN["adler32"]
    if zlib.ZLIB_RUNTIME_VERSION == GOLDEN["zlib_version"]:
        assert len(stream) == GOLDEN["level6_len"]
        assert hashlib.sha256(stream).hexdigest() == GOLDEN["level6_sha256"]


def test_oracle_on_golden(c0):
    raw, stream = c0
    assert oracle.adler32(raw) == GOLDEN["adler32"]
    out, status = oracle.decompress(stream, len(raw))
    assert status == 0 and hashlib.sha256(out).hexdigest() == GOLDEN["raw_sha256"]
    out, status = oracle.inflate_general(stream, len(raw))
    assert status == 0 and out == raw


@pytest.mark.gpu
def test_gpu_decodes_golden_stream(gpu, c0):
    from gpu_helpers import capi_decompress
    raw, stream = c0
    out, status, reserved = capi_decompress(stream, len(raw))
    assert (status, reserved) == (0, 0)
    assert hashlib.sha256(out).hexdigest() == GOLDEN["raw_sha256"]


@pytest.mark.gpu
def test_gpu_encodes_golden_raw(gpu, c0):
    from cuda_zlib import compress_zlib
    raw, _ = c0
    stream = compress_zlib(raw).cpu().numpy().tobytes()
    assert zlib.decompress(stream) == raw
    assert int.from_bytes(stream[-4:], "big") == GOLDEN["adler32"]
    assert len(stream) <= 1.02 * GOLDEN["level1_len"], (len(stream), GOLDEN["level1_len"])
