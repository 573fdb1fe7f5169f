import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")
    config.addinivalue_line("markers", "slow: long-running CPU test")


@pytest.fixture(scope="session")
def oracle():
    import oracle as o

    o.load()
    return o


@pytest.fixture(scope="session")
def gpu():
    """The spissa_amd package with a live default session; fails (never skips) without a GPU."""
    import ctypes

    import spissa_amd
    from spissa_amd import _ffi

    lib = _ffi.load()
    h = ctypes.c_void_p()
    st = lib.spissa_default_session(ctypes.byref(h))
    if st != 0:
        pytest.fail(f"no usable GPU for a gpu-marked test: {_ffi.last_error()}")
    print(f"[gpu] {lib.spissa_version().decode()} pid={os.getpid()}", flush=True)
    return spissa_amd
