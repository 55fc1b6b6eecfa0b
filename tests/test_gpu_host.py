"""Host-output decode: completed, read-only, byte-exact NumPy arrays.

Mirrors the reference's host tests (tests/test_host.py:70-141): bytes and
device-resident payloads, corruption and wrong extents raise CodecError and the
next call still succeeds, and a returned view stays valid after later decodes.
"""

import gc
import zlib

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _raw(size):
    block = bytes(range(251))
    return (block * ((size + len(block) - 1) // len(block)))[:size]


def _input(payload, resident):
    if not resident:
        return payload
    import torch
    return torch.from_numpy(np.frombuffer(payload, dtype=np.uint8).copy()).to("cuda:0")


@pytest.mark.parametrize("resident", [False, True], ids=["bytes", "resident"])
@pytest.mark.parametrize("size", [0, 65537, 1048576])
def test_host_array_is_completed_readonly_and_byte_exact(gpu, no_cpu_codec, resident, size):
    from cuda_zlib import decompress_zlib_host
    raw = _raw(size)
    payload = _input(zlib.compress(raw), resident)
    with no_cpu_codec:
        result = decompress_zlib_host(payload, size, 0)
    assert isinstance(result, np.ndarray)
    assert result.dtype == np.uint8 and result.shape == (size,)
    assert result.flags.c_contiguous and not result.flags.writeable
    assert memoryview(result).readonly
    assert memoryview(result) == memoryview(raw)


@pytest.mark.parametrize("resident", [False, True], ids=["bytes", "resident"])
@pytest.mark.parametrize("change", ["block-type", "truncated", "checksum", "short-output",
                                    "long-output"])
def test_host_decode_rejects_corruption_then_recovers(gpu, no_cpu_codec, resident, change):
    from cuda_zlib import CodecError, decompress_zlib_host
    raw = _raw(65537)
    valid = zlib.compress(raw)
    payload, expected = valid, len(raw)
    if change == "block-type":
        payload = valid[:2] + bytes(((valid[2] & ~6) | 6,)) + valid[3:]
    elif change == "truncated":
        payload = valid[:-6] + valid[-4:]
    elif change == "checksum":
        payload = valid[:-1] + bytes((valid[-1] ^ 1,))
    elif change == "short-output":
        expected -= 1
    else:
        expected += 1
    match = "Adler32 mismatch" if change == "checksum" else None
    with no_cpu_codec:
        with pytest.raises(CodecError, match=match):
            decompress_zlib_host(_input(payload, resident), expected, 0)
        recovered = decompress_zlib_host(_input(valid, resident), len(raw), 0)
    assert memoryview(recovered) == memoryview(raw)


def test_host_view_survives_gc_and_later_decode(gpu, no_cpu_codec):
    from cuda_zlib import decompress_zlib_host
    raw = _raw(1048576)
    second_raw = b"different output and extent" * 4096
    first_stream, second_stream = zlib.compress(raw), zlib.compress(second_raw)
    with no_cpu_codec:
        result = decompress_zlib_host(first_stream, len(raw), 0)
        view = memoryview(result)
        del result
        gc.collect()
        second = decompress_zlib_host(second_stream, len(second_raw), 0)
    assert memoryview(second) == memoryview(second_raw)
    del second
    gc.collect()
    assert view.readonly and view == memoryview(raw)
