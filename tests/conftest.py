import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


@pytest.fixture(scope="session")
def gpu():
    """The product library on device 0; fails (does not skip) when missing."""
    from arclight_amd import _lib, device
    _lib.load()
    n = device.device_count()
    assert n >= 1, "no GPU visible"
    info = device.device_info()
    print(f"\n[gpu] {info}", flush=True)
    return info
