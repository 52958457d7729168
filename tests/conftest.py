"""Shared fixtures.  GPU tests carry @pytest.mark.gpu; everything else runs on
the CPU (oracle checks, host logic, ABI load/export checks)."""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


@pytest.fixture(scope="session")
def wm():
    """The HIP library.  On a GPU run a missing build is an error, not a skip."""
    from whitematter_amd import _lib
    _lib.lib()
    _lib.call("wm_init", 0)
    return _lib


@pytest.fixture(scope="session")
def orc():
    import oracle
    return oracle
