import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device); runs the gfx950 kernels")


@pytest.fixture(scope="session")
def O():
    """The CPU oracle (oracle/tg_oracle.c through ctypes)."""
    from oracle import oracle
    oracle.lib()
    return oracle


@pytest.fixture(scope="session")
def tglib():
    """libtinygiant.so with device 0 initialised (GPU tests only)."""
    from tinygiant_amd._lib import call, require_lib
    lib = require_lib()
    call("tg_gpu_init", 0)
    return lib


def gpu_note(msg: str) -> None:
    """Print and flush what a GPU step is about to do (case name, shape)."""
    print(f"[gpu] {msg}", flush=True)
    sys.stdout.flush()
