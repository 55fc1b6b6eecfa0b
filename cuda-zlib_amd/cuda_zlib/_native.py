"""Loads the in-tree HIP codec library and binds its C ABI with ctypes.

The library (``libhip_zlib.so``, built from ``csrc/`` for gfx950) is the only
codec implementation: there is no CPU fallback.  A missing library raises
``BackendUnavailable`` at the first codec call.  Mirrors the reference's
native loader and pool controls (src/cuda_zlib/_ffi.py:21-41, 135-184).
"""

import ctypes
import os
import threading

from ._errors import BackendUnavailable

_LOCK = threading.Lock()
_LIBRARY = None
LIBRARY_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libhip_zlib.so")
INVALID_ARGUMENT = -1

_P = ctypes.c_void_p
_U64 = ctypes.c_uint64
_I64 = ctypes.c_int64
_I64P = ctypes.POINTER(ctypes.c_int64)

SIGNATURES = {
    "HipZlibCompress": [_P, _I64, _P, _U64, _P, _U64, _P, _U64],
    "HipZlibCompressNoAlloc": [_P, _I64, _P, _U64, _P, _U64, _P, _U64],
    "HipZlibCompressIndependent": [_P, _I64, _P, _U64, _P, _U64, _P, _U64],
    "HipZlibDecompress": [_P, _I64, _I64, _P, _U64, _P, _U64, _P, _U64],
    "HipZlibDecompressFormat": [_P, ctypes.c_int32, _P, _U64, _I64, _I64, _P, _U64, _P, _U64, _P,
                                _U64],
    "HipZlibCompressBatch": [_P, _I64, _I64P, _U64, _P, _U64, _P, _U64, _P, _U64, _U64],
    "HipZlibDecompressBatch": [_P, _I64P, _U64, _I64P, _U64, _P, _U64, _P, _U64, _U64, _P, _U64,
                               _P, _U64, _U64],
    "HipZlibSetWorkspaceRetention": [_U64],
    "HipZlibWorkspacePoolStats": [ctypes.c_int, ctypes.POINTER(_U64)],
    "HipZlibTrimWorkspacePool": [ctypes.c_int],
    "HipZlibErrorString": [ctypes.c_int],
    "HipZlibProfileEnable": [ctypes.c_int],
    "HipZlibProfileCollect": [ctypes.c_char_p, _U64, ctypes.c_int],
}


def workspace_retention():
    """Parse the pool release threshold from the environment (default 1 GiB)."""
    value = os.environ.get("CUDA_ZLIB_WORKSPACE_RETENTION_BYTES", str(1 << 30))
    if not value.isascii() or not value.isdecimal() or int(value) >= 1 << 64:
        raise ValueError("CUDA_ZLIB_WORKSPACE_RETENTION_BYTES must be an integer in [0, 2**64-1]")
    return int(value)


def _bind(library):
    for name, args in SIGNATURES.items():
        function = getattr(library, name)
        function.argtypes = args
        function.restype = (ctypes.c_char_p if name == "HipZlibErrorString" else
                            _U64 if name == "HipZlibProfileCollect" else ctypes.c_int)
    return library


def load(path=LIBRARY_PATH):
    """Load and bind the native library once per process."""
    global _LIBRARY
    with _LOCK:
        if _LIBRARY is None:
            retention = workspace_retention()
            # torch brings its own copy of the HIP runtime: load it first, so
            # that the codec library binds to the runtime torch's tensors and
            # streams belong to (loaded the other way round, the codec's calls
            # find no device).
            try:
                import torch  # noqa: F401
            except ImportError:
                pass
            if not os.path.exists(path):
                raise BackendUnavailable(
                    "native HIP codec library is not built (%s); run __graft_entry__.build()" % path)
            try:
                library = _bind(ctypes.CDLL(path))
            except OSError as exc:
                raise BackendUnavailable("native HIP codec library failed to load: %s" % exc) from exc
            check(library, library.HipZlibSetWorkspaceRetention(retention))
            _LIBRARY = library
        return _LIBRARY


def check(library, code):
    """Map a nonzero C-ABI return code to a Python exception."""
    if code == 0:
        return
    message = library.HipZlibErrorString(code)
    message = message.decode() if message else "unknown error"
    if code == INVALID_ARGUMENT:
        raise ValueError("native HIP codec: invalid argument: " + message)
    raise RuntimeError("native HIP codec: %s (HIP error %d)" % (message, code))


def int64_array(values):
    array = (ctypes.c_int64 * max(1, len(values)))(*values)
    return array


def profile_collect(library, reset=True):
    """{kernel: (launches, total_ms)} recorded while profiling was enabled."""
    size = library.HipZlibProfileCollect(None, 0, 0)
    buffer = ctypes.create_string_buffer(int(size) + 1)
    library.HipZlibProfileCollect(buffer, len(buffer), int(reset))
    result = {}
    for line in buffer.value.decode().splitlines():
        name, count, ms = line.split()
        result[name] = (int(count), float(ms))
    return result
