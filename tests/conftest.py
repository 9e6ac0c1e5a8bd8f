"""pytest configuration: import paths, the ``gpu`` marker, and the built library."""

from __future__ import annotations

import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for path in (ROOT, os.path.join(ROOT, "inf-engine_amd")):
    if path not in sys.path:
        sys.path.insert(0, path)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device); run with -m gpu")


@pytest.fixture(scope="session")
def native_lib():
    """The ctypes handle of libw4a16.so, building it first only if it is absent."""
    from w4a16 import _native

    if not os.path.exists(_native.LIB_PATH):
        from w4a16 import build

        build.build()
    return _native.load_library()
