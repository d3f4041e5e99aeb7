"""Test configuration.

Markers
- gpu: needs a ROCm GPU and libtrnsparse_hip.so; these are the parity tests
  of the HIP kernels against the CPU oracle (oracle/).
Everything else runs on the CPU (oracle pins, formats, host logic, the
C-ABI export check).
"""

from __future__ import annotations

import pathlib
import sys

import pytest

ROOT = pathlib.Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: requires a ROCm GPU (MI355X) and the built HIP library")


@pytest.fixture
def hip_backend():
    """Select the HIP backend for the test and check the native library loaded."""
    import trnsparse_amd as ts
    from trnsparse_amd.hip import _lib

    prev = ts.get_backend()
    ts.set_backend("hip")
    _lib.load()
    yield
    ts.set_backend(prev)


@pytest.fixture
def pytorch_backend():
    import trnsparse_amd as ts

    prev = ts.get_backend()
    ts.set_backend("pytorch")
    yield
    ts.set_backend(prev)
