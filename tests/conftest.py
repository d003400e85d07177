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
    if _library_stale(_lib.LIB_PATH):
        from hippo_leap_amd import build
        build.build()
    return _lib.load()


def _library_stale(lib_path: str) -> bool:
    """True when the library is missing or older than any kernel source or the
    public header, so that a test never runs a library built from old code."""
    if not os.path.exists(lib_path):
        return True
    built = os.path.getmtime(lib_path)
    csrc = os.path.join(ROOT, "hippo_leap_amd", "csrc")
    sources = [os.path.join(csrc, f) for f in os.listdir(csrc)]
    sources.append(os.path.join(ROOT, "include", "hl_attn.h"))
    return any(os.path.getmtime(s) > built for s in sources if os.path.isfile(s))


@pytest.fixture(scope="session")
def orc():
    import oracle
    if not os.path.exists(oracle.LIB_PATH):
        oracle.build()
    oracle.lib()
    return oracle
