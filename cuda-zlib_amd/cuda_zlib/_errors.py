"""Errors distinguish malformed input from unavailable/unsupported backends.

Same three classes and base classes as the reference (src/cuda_zlib/_errors.py:6-16),
so callers' ``except`` clauses keep working unchanged.
"""


class CodecError(ValueError):
    """Malformed stream, checksum/extent mismatch, or codec workspace limit."""


class BackendUnavailable(NotImplementedError):
    """The requested GPU device, native library or optional runtime is unavailable."""


class UnsupportedStream(NotImplementedError):
    """Valid wrapper features outside this bounded implementation's subset."""
