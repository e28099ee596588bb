import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) device and libmanta_rocm.so")
    config.addinivalue_line("markers", "slow: full-size BASELINE configuration")


@pytest.fixture(scope="session")
def rt():
    """One runtime per test session (GPU tests only).  No skip: a GPU test
    run on a machine without the library or the device fails loudly."""
    from manta_amd import rocm

    r = rocm.Runtime(0)
    yield r
    r.close()
