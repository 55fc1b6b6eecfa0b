"""Device-explicit convenience API: the same calls with a required ``device=``.

Counterpart of the reference's ``cuda_zlib.jax`` module (src/cuda_zlib/jax.py:10-34),
which requires a JAX device; here the device must be a ``torch.device``.
"""

from . import _codec
from ._errors import BackendUnavailable


def _admit(device):
    _codec._validate_device(device)
    if type(device) is int:
        raise BackendUnavailable("torch GPU device required")
    return device


def decompress_zlib(payload, expected_bytes, *, device):
    _admit(device)
    return _codec.decompress_zlib(payload, expected_bytes, device)


def compress_zlib(data, *, device, chunk_bytes=32768):
    _admit(device)
    return _codec.compress_zlib(data, device, chunk_bytes=chunk_bytes)


def compress_zlib_padded(data, *, device, chunk_bytes=32768):
    _admit(device)
    return _codec.compress_zlib_padded(data, device, chunk_bytes=chunk_bytes)


def decompress_zlib_checked(payload, expected_bytes, *, device):
    _admit(device)
    return _codec.decompress_zlib_checked(payload, expected_bytes, device)
