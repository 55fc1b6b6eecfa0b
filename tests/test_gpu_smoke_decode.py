"""First GPU checks of the serial small-stream route against CPU zlib."""

import random
import zlib

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _decode(payload, size, device):
    import cuda_zlib
    out, meta = cuda_zlib.decompress_zlib_checked(payload, size, device)
    return out.cpu().numpy().tobytes(), [int(v) for v in meta.cpu().numpy()]


@pytest.mark.parametrize("level", [0, 1, 6, 9])
@pytest.mark.parametrize("kind", ["text", "random", "zeros", "empty"])
def test_small_route_matches_zlib(gpu, no_cpu_codec, level, kind):
    rng = random.Random(7)
    if kind == "text":
        raw = b"".join(rng.choice([b"alpha ", b"beta ", b"gamma ", b"delta\n"]) for _ in range(5000))
    elif kind == "random":
        raw = rng.randbytes(40000)
    elif kind == "zeros":
        raw = bytes(65536)
    else:
        raw = b""
    payload = zlib.compress(raw, level)
    with no_cpu_codec:
        data, meta = _decode(payload, len(raw), gpu)
    assert meta == [0, 0]
    assert data == raw


def test_small_route_adler_and_size_errors(gpu):
    raw = b"a checked stream\x00" * 200
    payload = zlib.compress(raw, 6)
    bad = payload[:-1] + bytes([payload[-1] ^ 1])
    data, meta = _decode(bad, len(raw), gpu)
    assert meta == [21, 0] and data == raw
    _, meta = _decode(payload, len(raw) + 1, gpu)
    assert meta == [11, 0]
    _, meta = _decode(payload, len(raw) - 1, gpu)
    assert meta == [7, 0]
    import torch
    bad_header = torch.frombuffer(bytearray(b"\x00" + payload[1:]), dtype=torch.uint8).to("cuda")
    data, meta = _decode(bad_header, len(raw), gpu)
    assert meta == [15, 0] and data == bytes(len(raw))
