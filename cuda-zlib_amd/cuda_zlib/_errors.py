"""Exception classes of the codec.

Three classes, with the reference's names and base classes
(src/cuda_zlib/_errors.py:6-16), so that ``except`` clauses written against
the reference catch the same failures here:

- ``CodecError`` (a ``ValueError``): the data is wrong -- a corrupt or
  truncated stream, a checksum or size that does not match, or a workspace
  bound that the stream exceeds.
- ``BackendUnavailable`` (a ``NotImplementedError``): the code cannot run --
  no ROCm device, no torch, or the native library is not built.
- ``UnsupportedStream`` (a ``NotImplementedError``): the stream is well formed
  but uses a wrapper feature the called entry point does not decode.
"""


class CodecError(ValueError):
    """The stream, its checksum or its declared size is wrong, or a workspace bound was hit."""


class BackendUnavailable(NotImplementedError):
    """No usable ROCm device, torch build or native codec library."""


class UnsupportedStream(NotImplementedError):
    """A well-formed stream whose wrapper feature this entry point does not decode."""
