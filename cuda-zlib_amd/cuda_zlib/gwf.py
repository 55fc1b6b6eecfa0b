"""Decoding of compressed GWF frame vectors (FrVect) on the GPU.

Counterpart of the reference's PyCBC adapter
(integrations/pycbc/gwf_deflate_jax.py:1-55), which hands a frame vector's
zlib payload to the codec and reinterprets the bytes as the vector's samples.
That adapter imports its frame types from a module the reference does not
ship; this one carries the little it needs itself: the vector record, the
compression and sample-type codes of the frame format, and the two error
classes, with the reference's mapping of codec errors onto them.

Frame-format codes used here (the IGWD frame specification's FrVect):

- ``compress``: the low byte is the method -- 0 raw, 1 "gzip" (a zlib
  stream), 3 differences then "gzip"; the flag 0x100 marks little-endian
  samples (without it the samples are big-endian).
- ``type``: 0 int8, 1 int16, 2 float64, 3 float32, 4 int32, 5 int64,
  6 complex64, 7 complex128, 8 string, 9 uint16, 10 uint32, 11 uint64,
  12 uint8.

Decoded samples are returned as a torch tensor on the GPU in native
(little-endian) byte order.
"""

import enum
from dataclasses import dataclass

import numpy as np

from . import _codec
from ._errors import BackendUnavailable, CodecError, UnsupportedStream


class GWFFormatError(ValueError):
    """The frame vector's payload or header is malformed."""


class GWFDeflateUnavailable(NotImplementedError):
    """The vector cannot be decoded here: no GPU backend, or a method or type it does not cover."""


class CompressionKind(enum.IntEnum):
    RAW = 0
    GZIP = 1
    DIFF_GZIP = 3


LITTLE_ENDIAN_FLAG = 0x100
STRING_TYPE = 8

# type code -> NumPy sample type (little-endian form)
SAMPLE_TYPES = {
    0: np.dtype("<i1"), 1: np.dtype("<i2"), 2: np.dtype("<f8"), 3: np.dtype("<f4"),
    4: np.dtype("<i4"), 5: np.dtype("<i8"), 6: np.dtype("<c8"), 7: np.dtype("<c16"),
    9: np.dtype("<u2"), 10: np.dtype("<u4"), 11: np.dtype("<u8"), 12: np.dtype("<u1"),
}


@dataclass(frozen=True)
class FrVect:
    """The fields of a frame vector that decoding needs."""

    compress: int
    type_code: int
    n_data: int
    payload: bytes

    @property
    def kind(self):
        method = self.compress & 0xFF
        try:
            return CompressionKind(method)
        except ValueError:
            raise GWFDeflateUnavailable("frame compression method %d is not decoded here" % method)

    @property
    def little_endian(self):
        return bool(self.compress & LITTLE_ENDIAN_FLAG)

    @property
    def dtype(self):
        if self.type_code not in SAMPLE_TYPES:
            raise GWFDeflateUnavailable("frame vector type %d has no numeric samples" % self.type_code)
        return SAMPLE_TYPES[self.type_code]

    @property
    def nbytes(self):
        return self.n_data * self.dtype.itemsize


def decompress_zlib(payload, expected_bytes, device=0):
    """``cuda_zlib.decompress_zlib`` with the frame adapter's exceptions.

    A corrupt stream raises ``GWFFormatError``.  A stream the codec does not
    decode raises ``GWFDeflateUnavailable``, except a preset-dictionary
    stream, which frame files never contain and so is a format error.  A
    missing GPU backend raises ``GWFDeflateUnavailable``.
    """
    try:
        return _codec.decompress_zlib(payload, expected_bytes, device)
    except CodecError as exc:
        raise GWFFormatError(str(exc)) from exc
    except UnsupportedStream as exc:
        dictionary = isinstance(payload, bytes) and len(payload) > 1 and bool(payload[1] & 0x20)
        if dictionary:
            raise GWFFormatError(str(exc)) from exc
        raise GWFDeflateUnavailable(str(exc)) from exc
    except BackendUnavailable as exc:
        raise GWFDeflateUnavailable(str(exc)) from exc


def compile_kernels(device=0):
    """Load the codec for ``device`` ahead of the first frame decode."""
    try:
        _codec.compile_kernels(device)
    except BackendUnavailable as exc:
        raise GWFDeflateUnavailable(str(exc)) from exc


def _torch_dtype(dtype):
    import torch
    table = {"i1": torch.int8, "i2": torch.int16, "i4": torch.int32, "i8": torch.int64,
             "u1": torch.uint8, "u2": torch.uint16, "u4": torch.uint32, "u8": torch.uint64,
             "f4": torch.float32, "f8": torch.float64, "c8": torch.complex64,
             "c16": torch.complex128}
    return table[dtype.str[1:]]


def samples_from_bytes(raw, vector):
    """Reinterpret decoded bytes (a device uint8 tensor) as the vector's samples.

    Big-endian samples are byte-swapped on the device; differenced integer
    samples are summed back (with the wrap-around of their width).
    """
    import torch
    dtype = vector.dtype
    size = dtype.itemsize
    if raw.numel() != vector.nbytes:
        raise GWFFormatError("decoded %d bytes for %d samples of %d bytes"
                             % (raw.numel(), vector.n_data, size))
    if not vector.little_endian and size > 1:
        # Complex samples swap each of their two components.
        part = size // 2 if dtype.kind == "c" else size
        raw = raw.view(-1, part).flip(1).reshape(-1)
    samples = raw.view(_torch_dtype(dtype))
    if vector.kind == CompressionKind.DIFF_GZIP:
        if dtype.kind not in "iu":
            raise GWFDeflateUnavailable("differenced samples must be integers")
        bits = 8 * size
        total = torch.cumsum(samples.to(torch.int64), 0)
        if bits < 64:
            total = torch.remainder(total, 1 << bits)
            if dtype.kind == "i":
                total = torch.where(total >= (1 << (bits - 1)), total - (1 << bits), total)
        samples = total.to(_torch_dtype(dtype))
    return samples


def decode_fr_vect_deflate(vector, device=0):
    """Decode a zlib-compressed frame vector on the GPU; returns its samples.

    Accepts the "gzip" and differenced "gzip" methods of numeric vectors
    (the reference's adapter takes the first of them, reference
    integrations/pycbc/gwf_deflate_jax.py:47-55).
    """
    if vector.type_code == STRING_TYPE:
        raise GWFDeflateUnavailable("string vectors are not decoded on the GPU")
    if vector.kind not in (CompressionKind.GZIP, CompressionKind.DIFF_GZIP):
        raise GWFDeflateUnavailable("frame vector is not zlib-compressed")
    raw = decompress_zlib(vector.payload, vector.nbytes, device)
    return samples_from_bytes(raw, vector)


def encode_fr_vect_deflate(samples, type_code, *, little_endian=True, difference=False,
                           device=0, chunk_bytes=32768):
    """Compress samples (a NumPy array) into a frame vector with the GPU encoder.

    The inverse of ``decode_fr_vect_deflate``: the samples are laid out in the
    requested byte order (differenced first when asked), compressed on the
    GPU, and returned as an ``FrVect`` whose payload is the zlib stream.
    """
    dtype = SAMPLE_TYPES[type_code]
    values = np.ascontiguousarray(samples, dtype=dtype)
    if difference:
        if dtype.kind not in "iu":
            raise GWFDeflateUnavailable("differenced samples must be integers")
        values = np.diff(values, prepend=values.dtype.type(0)).astype(dtype)
    if not little_endian:
        values = values.astype(dtype.newbyteorder(">"))
    stream = _codec.compress_zlib(values.tobytes(), device, chunk_bytes=chunk_bytes)
    method = CompressionKind.DIFF_GZIP if difference else CompressionKind.GZIP
    compress = int(method) | (LITTLE_ENDIAN_FLAG if little_endian else 0)
    return FrVect(compress, type_code, int(values.size), stream.cpu().numpy().tobytes())
