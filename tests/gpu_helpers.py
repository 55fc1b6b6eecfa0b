"""Direct C-ABI calls for GPU tests (bypassing Python-side validation)."""

import ctypes

MAX = 262144


def _tensor(data, device):
    import numpy as np
    import torch
    host = torch.from_numpy(np.frombuffer(bytes(data), dtype=np.uint8).copy())
    return host.to(device)


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr() if t.numel() else 0)


def capi_decompress(payload, expected, max_candidates=MAX, max_blocks=MAX, device=0):
    """HipZlibDecompress through ctypes; returns (output bytes, status, reserved)."""
    import torch
    from cuda_zlib import _native
    lib = _native.load()
    dev = torch.device("cuda", device)
    inp = _tensor(payload, dev)
    out = torch.empty(expected, dtype=torch.uint8, device=dev)
    meta = torch.full((2,), 0xDEAD, dtype=torch.uint32, device=dev)
    stream = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    rc = lib.HipZlibDecompress(stream, max_candidates, max_blocks, _ptr(inp), len(payload),
                               _ptr(out), expected, _ptr(meta), 2)
    _native.check(lib, rc)
    torch.cuda.synchronize(dev)
    m = meta.cpu().numpy()
    return out.cpu().numpy().tobytes(), int(m[0]), int(m[1])
