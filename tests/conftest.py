import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


@pytest.fixture(scope="session")
def hl():
    """The attention library (built in-tree if missing; no CPU fallback)."""
    from hippo_leap_amd import _lib
    if not os.path.exists(_lib.LIB_PATH):
        from hippo_leap_amd import build
        build.build()
    return _lib.load()


@pytest.fixture(scope="session")
def orc():
    import oracle
    if not os.path.exists(oracle.LIB_PATH):
        oracle.build()
    oracle.lib()
    return oracle
