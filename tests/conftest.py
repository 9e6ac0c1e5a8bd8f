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
    """The ctypes handle of libw4a16.so, (re)building it first when it is absent
    or older than its sources (and hipcc is there to build it)."""
    from w4a16 import _native, build

    if build.is_stale() and (os.path.exists(build.HIPCC) or not os.path.exists(_native.LIB_PATH)):
        build.build()
    return _native.load_library()
