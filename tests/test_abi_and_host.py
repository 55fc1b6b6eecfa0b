"""CPU checks of the C-ABI library and the host-side API (no GPU calls).

The library must load without a GPU and export every entry point that
include/hip_zlib.h declares; the Python layer must validate arguments before
it touches torch or the device, as the reference's host layer does
(src/cuda_zlib/_codec.py:53-148, tests/test_host.py:47-67).
"""

import builtins
import ctypes
import os
import re

import pytest

from conftest import ROOT

HEADER = os.path.join(ROOT, "include", "hip_zlib.h")


def _declared():
    text = open(HEADER).read()
    return re.findall(r"^\s*(?:int|uint64_t|const char\s*\*)\s*(HipZlib\w+)\s*\(", text, re.M)


def _torch_first():
    """torch brings its own HIP runtime: it must be loaded before the codec
    library, or a later GPU test in this process finds no device."""
    try:
        import torch  # noqa: F401
    except ImportError:
        pass


def test_library_exports_every_declared_entry_point():
    from cuda_zlib import _native
    assert os.path.exists(_native.LIBRARY_PATH), "build the library first (__graft_entry__.build())"
    _torch_first()
    lib = ctypes.CDLL(_native.LIBRARY_PATH)
    names = _declared()
    assert len(names) >= 10
    for name in names:
        assert hasattr(lib, name), name
    assert set(names) == set(_native.SIGNATURES)


def test_error_strings_need_no_device():
    from cuda_zlib import _native
    _torch_first()
    lib = _native._bind(ctypes.CDLL(_native.LIBRARY_PATH))
    assert lib.HipZlibErrorString(1)  # a HIP error code maps to its runtime message
    assert lib.HipZlibErrorString(-1) is not None


def test_retention_environment_parsing(monkeypatch):
    from cuda_zlib import _native
    monkeypatch.setenv("CUDA_ZLIB_WORKSPACE_RETENTION_BYTES", "12345")
    assert _native.workspace_retention() == 12345
    for bad in ("-1", "1e9", str(1 << 64), "x"):
        monkeypatch.setenv("CUDA_ZLIB_WORKSPACE_RETENTION_BYTES", bad)
        with pytest.raises(ValueError):
            _native.workspace_retention()


@pytest.mark.parametrize("payload,expected,error", [
    (b"", 0, "CodecError"),
    (b"\x78\x00" + b"\x00" * 8, 0, "CodecError"),
    (b"\x1f\x8b" + b"\x00" * 8, 0, "UnsupportedStream"),
    (b"", -1, "ValueError"),
    (b"", True, "ValueError"),
    (b"", 2**32, "ValueError"),
])
def test_host_rejects_invalid_input_before_loading_torch(monkeypatch, payload, expected, error):
    import cuda_zlib
    actual_import = builtins.__import__

    def guarded(name, *args, **kwargs):
        if name.split(".")[0] == "torch":
            pytest.fail("invalid host input loaded the GPU backend")
        return actual_import(name, *args, **kwargs)

    monkeypatch.setattr(builtins, "__import__", guarded)
    exc = getattr(cuda_zlib, error, None) or getattr(builtins, error)
    with pytest.raises(exc):
        cuda_zlib.decompress_zlib_host(payload, expected)


def test_preset_dictionary_header_is_unsupported():
    import cuda_zlib
    cmf, flg = 0x78, 0x20
    flg += (31 - (cmf * 256 + flg) % 31) % 31
    with pytest.raises(cuda_zlib.UnsupportedStream):
        cuda_zlib.decompress_zlib_host(bytes((cmf, flg)) + b"\x00" * 8, 0)


@pytest.mark.parametrize("chunk", [255, 65536, 1.5, True])
def test_compress_rejects_chunk_sizes(chunk):
    import cuda_zlib
    with pytest.raises(ValueError):
        cuda_zlib.compress_zlib_padded(b"abc", chunk_bytes=chunk)


def test_batch_size_validation():
    import cuda_zlib
    with pytest.raises(ValueError):
        cuda_zlib.compress_zlib_batch_padded(b"", ())
    with pytest.raises(ValueError):
        cuda_zlib.compress_zlib_batch_padded(b"abc", (2,))
    with pytest.raises(ValueError):
        cuda_zlib.compress_zlib_batch_padded(b"abc", (-1, 4))
    with pytest.raises(ValueError):
        cuda_zlib.decompress_zlib_batch_checked(b"abcdefgh", (8,), (1, 2))


def test_capacity_formula_matches_the_reference():
    from cuda_zlib import _codec
    # n + 5 * max(1, ceil(n / chunk)) + 6 (reference _codec.py:151-166).
    assert _codec._capacity(0, 32768) == (1, 11)
    assert _codec._capacity(32768, 32768) == (1, 32768 + 11)
    assert _codec._capacity(32769, 32768) == (2, 32769 + 16)
    assert _codec._batch_capacities((0, 100, 70000), 32768) == (11, 111, 70000 + 21)


def test_status_table_is_complete():
    from cuda_zlib import _codec
    # 0-23 are the reference's; 24 and 25 belong to the gzip / dictionary entry points.
    assert sorted(_codec._MESSAGES) == [s for s in range(26) if s != 8]
    assert _codec._MESSAGES[21].endswith("Adler32 mismatch")


def test_oracle_not_imported_by_the_package():
    pkg = os.path.join(ROOT, "cuda-zlib_amd")
    for dirpath, _, files in os.walk(pkg):
        for f in files:
            if f.endswith((".py", ".hip", ".h", ".cpp")):
                text = open(os.path.join(dirpath, f)).read()
                assert "oracle" not in text.lower(), f


def test_retention_can_be_set_and_read_without_a_device():
    """Before any pool exists the controls touch no GPU: set, then read back."""
    import subprocess
    import sys
    script = (
        "import ctypes, sys; sys.path[:0] = [%r]\n"
        "from cuda_zlib import _native\n"
        "lib = _native._bind(ctypes.CDLL(_native.LIBRARY_PATH))\n"
        "assert lib.HipZlibSetWorkspaceRetention(12345) == 0\n"
        "stats = (ctypes.c_uint64 * 4)()\n"
        "assert lib.HipZlibWorkspacePoolStats(0, stats) == 0\n"
        "assert list(stats) == [12345, 0, 0, 0], list(stats)\n"
        "assert lib.HipZlibTrimWorkspacePool(0) == 0\n"
        "assert lib.HipZlibWorkspacePoolStats(0, None) == _native.INVALID_ARGUMENT\n"
        % os.path.join(ROOT, "cuda-zlib_amd"))
    proc = subprocess.run([sys.executable, "-c", script], capture_output=True, text=True,
                          timeout=120, env=dict(os.environ, HIP_VISIBLE_DEVICES=""))
    assert proc.returncode == 0, proc.stderr
