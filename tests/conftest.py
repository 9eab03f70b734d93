import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) device")
    config.addinivalue_line("markers", "slow: long-running CPU pinning check")


@pytest.fixture(scope="session")
def oracle_lib():
    import oracle
    oracle.build()
    return oracle


@pytest.fixture(scope="session")
def hip():
    """The product library on a real device (GPU tests only)."""
    from tokenvector.inference_amd import _lib
    L = _lib.lib()
    n = L.tkv_hip_device_count()
    assert n >= 1, "no gfx950 device visible: GPU tests need an MI355X"
    return _lib
