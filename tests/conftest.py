"""Shared test configuration.

`gpu` tests run the gfx950 library through its C ABI and check it against the
CPU oracle; everything else runs on the CPU (oracle pins, host logic, ABI
exports).  GPU tests fail loudly when the library or the device is missing.
"""
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def gpu():
    """The loaded library on a visible gfx950 device (hard failure otherwise)."""
    import torch

    from deltafin_amd import _lib

    assert torch.cuda.is_available(), "GPU test run without a visible HIP device"
    lib = _lib.load()
    rc = lib.k3_hip_moe_available(0)
    assert rc == 1, f"k3_hip_moe_available(0) = {rc}: {_lib.last_error()}"
    torch.cuda.init()
    return lib
