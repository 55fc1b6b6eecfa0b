"""Host-output decoding: ``decompress_zlib_host`` and ``decompress_zlib_batch_host``.

The contract checked here (the reference states it in src/cuda_zlib/_codec.py:431-448):
the result is a finished NumPy uint8 array in pinned host memory, read-only,
equal to the source bytes; a failing stream raises ``CodecError`` carrying the
status the oracle gives it, and the next call on the same device works; a
returned array keeps its own storage however many decodes follow.

Inputs come from the seeded workload generators; failures are built with the
test writer and checked against the oracle's status, so every expected status
is the oracle's, never a literal copied from elsewhere.
"""

import gc
import hashlib
import re
import warnings
import zlib

import numpy as np
import pytest

import deflate_writer as dw
import workloads
from oracle import oracle

pytestmark = pytest.mark.gpu

STATUS = re.compile(r"\(Deflate status (\d+)\)")


def _text(size, seed):
    return workloads.text_like(size, np.random.default_rng(seed))


def _as_device(payload):
    import torch
    return torch.frombuffer(bytearray(payload), dtype=torch.uint8).to("cuda:0")


# Sizes on both sides of the serial route's 64 KiB output bound, and empty output.
@pytest.mark.parametrize("size", [0, 1, 4093, 65536, 65537, 3 << 20])
@pytest.mark.parametrize("on_device", [False, True], ids=["host-bytes", "device-tensor"])
def test_result_is_a_finished_readonly_pinned_copy(gpu, no_cpu_codec, size, on_device):
    import torch
    from cuda_zlib import decompress_zlib_host
    raw = _text(size, 100 + size)
    stream = zlib.compress(raw, 9)
    payload = _as_device(stream) if on_device else stream
    with no_cpu_codec:
        array = decompress_zlib_host(payload, size, 0)
    # No stream synchronisation here: the array must already be complete.
    assert type(array) is np.ndarray
    assert array.dtype == np.uint8 and array.ndim == 1 and array.size == size
    assert array.flags.c_contiguous and not array.flags.writeable
    with pytest.raises(ValueError):
        array[:1] = 0
    assert array.tobytes() == raw
    if size:
        with warnings.catch_warnings():  # torch warns about wrapping a read-only array
            warnings.simplefilter("ignore")
            assert torch.from_numpy(array).is_pinned()


def _failures():
    """(name, stream, declared size) triples that the oracle rejects."""
    raw = _text(90000, 7)
    good = zlib.compress(raw, 6)
    cases = [
        ("adler", good[:-4] + (zlib.adler32(raw) ^ 0x00010000).to_bytes(4, "big"), len(raw)),
        ("declared-short", good, len(raw) - 1),
        ("declared-long", good, len(raw) + 1),
        ("reserved-type", dw.wrap(b"\x07" + b"\x00" * 5, b""), 0),
        ("truncated-body", good[:len(good) // 2] + good[-4:], len(raw)),
        ("stored-nlen", dw.wrap(b"\x01\x05\x00\xfa\xfe" + b"abcde", b"abcde"), 5),
        ("header-check", bytes((0x78, 0x9d)) + good[2:], len(raw)),
    ]
    return cases


@pytest.mark.parametrize("case", _failures(), ids=lambda c: c[0])
def test_failure_raises_the_oracle_status_then_the_device_recovers(gpu, no_cpu_codec, case):
    from cuda_zlib import CodecError, decompress_zlib_host
    _, stream, declared = case
    _, want = oracle.decompress(stream, declared)
    assert want != 0
    after = _text(70000, 8)
    after_stream = zlib.compress(after, 1)
    with no_cpu_codec:
        with pytest.raises(CodecError) as info:
            decompress_zlib_host(_as_device(stream), declared, 0)
        recovered = decompress_zlib_host(after_stream, len(after), 0)
    found = STATUS.search(str(info.value))
    assert found is not None and int(found.group(1)) == want
    assert recovered.tobytes() == after


def test_arrays_keep_their_storage_across_many_later_decodes(gpu, no_cpu_codec):
    from cuda_zlib import decompress_zlib_host
    sizes = [1 << 20, 300000, 65536, 5000]
    raws = [_text(n, 40 + i) for i, n in enumerate(sizes)]
    streams = [zlib.compress(r, 6) for r in raws]
    digests = [hashlib.sha256(r).hexdigest() for r in raws]
    kept = []
    with no_cpu_codec:
        for stream, raw in zip(streams, raws):
            kept.append(memoryview(decompress_zlib_host(stream, len(raw), 0)))
        # Churn the pinned allocator: results of the same sizes, dropped at once.
        for _ in range(3):
            for stream, raw in zip(streams[::-1], raws[::-1]):
                decompress_zlib_host(stream, len(raw), 0)
            gc.collect()
    for view, digest in zip(kept, digests):
        assert view.readonly
        assert hashlib.sha256(view).hexdigest() == digest


def test_batch_views_share_one_buffer_that_outlives_its_siblings(gpu, no_cpu_codec):
    from cuda_zlib import decompress_zlib_batch_host
    raws = [_text(n, 60 + n % 97) for n in (0, 17, 4096, 70000, 200000)]
    streams = [zlib.compress(r, 6) for r in raws]
    with no_cpu_codec:
        views = decompress_zlib_batch_host(streams, [len(r) for r in raws], 0)
    assert len(views) == len(raws)
    for view, raw in zip(views, raws):
        assert view.dtype == np.uint8 and not view.flags.writeable
        assert view.tobytes() == raw
    last = views[-1]
    del views
    gc.collect()
    with no_cpu_codec:
        decompress_zlib_batch_host(streams[::-1], [len(r) for r in raws[::-1]], 0)
    assert last.tobytes() == raws[-1]
