"""Test configuration: import paths, the ``gpu`` marker and shared fixtures."""

import os
import sys
import zlib

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for path in (os.path.join(ROOT, "cuda-zlib_amd"), ROOT, os.path.dirname(os.path.abspath(__file__))):
    if path not in sys.path:
        sys.path.insert(0, path)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU and the built HIP library")


@pytest.fixture(scope="session")
def gpu():
    """Index of the GPU under test; skips when no ROCm device is visible."""
    torch = pytest.importorskip("torch")
    if not torch.cuda.is_available() or torch.version.hip is None:
        pytest.skip("no ROCm GPU visible")
    return 0


@pytest.fixture
def no_cpu_codec(monkeypatch):
    """Fail the test if anything calls CPU zlib while the guard is active."""
    def forbidden(*args, **kwargs):
        raise AssertionError("CPU zlib called during a GPU codec call")

    class Guard:
        def __enter__(self):
            self._ctx = monkeypatch.context()
            patch = self._ctx.__enter__()
            for name in ("compress", "decompress", "compressobj", "decompressobj"):
                patch.setattr(zlib, name, forbidden)
            return self

        def __exit__(self, *exc):
            return self._ctx.__exit__(*exc)

    return Guard()
