"""C-ABI calls with input and output pointers at odd byte offsets.

The entry points take plain device pointers; nothing in the interface asks
for alignment, so every kernel must handle buffers that start at any byte.
Each buffer here lies inside a larger allocation filled with a guard byte,
and the bytes around the output must come back untouched.
"""

import ctypes
import zlib

import numpy as np
import pytest

import workloads
from gpu_helpers import _ptr

pytestmark = pytest.mark.gpu

GUARD = 0xAB
OFFSETS = [(1, 3), (3, 1), (7, 13), (0, 5), (5, 0)]


def _lib():
    from cuda_zlib import _native
    return _native, _native.load()


def _stream():
    import torch
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _at(t, off):
    return ctypes.c_void_p(t.data_ptr() + off)


def _placed(data, off, pad=64):
    """A guard-filled device buffer holding `data` at byte `off`."""
    import torch
    host = np.full(off + len(data) + pad, GUARD, np.uint8)
    host[off:off + len(data)] = np.frombuffer(data, np.uint8)
    return torch.from_numpy(host).cuda()


def _guarded(size, off, pad=64):
    import torch
    return torch.full((off + size + pad,), GUARD, dtype=torch.uint8, device="cuda")


def _cases():
    text = workloads.text_like(3 << 20, np.random.default_rng(31))
    small = workloads.text_like(10000, np.random.default_rng(32))
    rand = np.random.default_rng(33).integers(0, 256, 200000, dtype=np.uint8).tobytes()
    return [("text-3MiB-l6", text, zlib.compress(text, 6)),
            ("text-10KB-l6", small, zlib.compress(small, 6)),
            ("stored-200KB", rand, zlib.compress(rand, 0))]


@pytest.mark.parametrize("in_off,out_off", OFFSETS)
def test_decompress_at_odd_offsets(gpu, in_off, out_off):
    import torch
    native, lib = _lib()
    for name, raw, stream in _cases():
        inp = _placed(stream, in_off)
        out = _guarded(len(raw), out_off)
        meta = torch.full((2,), 0xDEAD, dtype=torch.uint32, device="cuda")
        native.check(lib, lib.HipZlibDecompress(_stream(), 262144, 262144, _at(inp, in_off),
                                                len(stream), _at(out, out_off), len(raw),
                                                _ptr(meta), 2))
        host = out.cpu().numpy()
        assert meta.cpu().numpy().tolist() == [0, 0], name
        assert host[out_off:out_off + len(raw)].tobytes() == raw, name
        assert (host[:out_off] == GUARD).all() and (host[out_off + len(raw):] == GUARD).all(), name


@pytest.mark.parametrize("in_off,out_off", OFFSETS)
def test_compress_at_odd_offsets(gpu, in_off, out_off):
    import torch
    native, lib = _lib()
    for name, raw, _ in _cases():
        cap = len(raw) + 5 * max(1, (len(raw) + 32767) // 32768) + 6
        inp = _placed(raw, in_off)
        out = _guarded(cap, out_off)
        meta = torch.full((2,), 0xDEAD, dtype=torch.uint32, device="cuda")
        native.check(lib, lib.HipZlibCompress(_stream(), 32768, _at(inp, in_off), len(raw),
                                              _at(out, out_off), cap, _ptr(meta), 2))
        host = out.cpu().numpy()
        length, status = meta.cpu().numpy().tolist()
        assert status == 0, name
        assert zlib.decompress(host[out_off:out_off + length].tobytes()) == raw, name
        # The slot past the stream is zeroed up to its capacity, and not beyond.
        assert not host[out_off + length:out_off + cap].any(), name
        assert (host[:out_off] == GUARD).all() and (host[out_off + cap:] == GUARD).all(), name


@pytest.mark.parametrize("in_off,out_off", OFFSETS[:3])
def test_batches_at_odd_offsets(gpu, in_off, out_off):
    import torch
    from cuda_zlib._native import int64_array
    native, lib = _lib()
    rng = np.random.default_rng(34)
    raws = [workloads.text_like(int(n), rng) for n in rng.integers(0, 40000, 37)]
    raws[5] = b""
    sizes = [len(r) for r in raws]
    caps = [s + 5 * max(1, (s + 32767) // 32768) + 6 for s in sizes]
    blob = b"".join(raws)
    n = len(raws)
    inp = _placed(blob, in_off)
    slots = _guarded(sum(caps), out_off)
    emeta = torch.zeros(n * 2, dtype=torch.uint32, device="cuda")
    native.check(lib, lib.HipZlibCompressBatch(
        _stream(), 32768, int64_array(sizes), n, _at(inp, in_off), len(blob), _at(slots, out_off),
        sum(caps), _ptr(emeta), n, 2))
    em = emeta.view(n, 2).cpu().numpy()
    assert not em[:, 1].any()
    host = slots.cpu().numpy()
    assert (host[:out_off] == GUARD).all() and (host[out_off + sum(caps):] == GUARD).all()
    at = out_off
    for r, c, (length, _) in zip(raws, caps, em.tolist()):
        assert zlib.decompress(host[at:at + length].tobytes()) == r
        at += c
    # Decode the slots in place from an odd offset into an odd offset.
    out = _guarded(len(blob), in_off)
    dmeta = torch.full((n * 2,), 0xDEAD, dtype=torch.uint32, device="cuda")
    native.check(lib, lib.HipZlibDecompressBatch(
        _stream(), int64_array(caps), n, int64_array(sizes), n, _at(slots, out_off), sum(caps),
        _ptr(emeta), n, 2, _at(out, in_off), len(blob), _ptr(dmeta), n, 2))
    dm = dmeta.view(n, 2).cpu().numpy()
    assert not dm[:, 0].any()
    got = out.cpu().numpy()
    assert got[in_off:in_off + len(blob)].tobytes() == blob
    assert (got[:in_off] == GUARD).all() and (got[in_off + len(blob):] == GUARD).all()
