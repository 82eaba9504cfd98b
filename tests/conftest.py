"""Shared fixtures.  Tests marked ``gpu`` need an MI355X (gfx950); the rest
run on the CPU (oracle, host logic, ABI surface)."""
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a gfx950 GPU")
    config.addinivalue_line("markers", "slow: takes more than a few seconds")


@pytest.fixture(scope="session")
def dev():
    """Device 0, opened.  A GPU test without a GPU fails: nothing falls back."""
    import accel_amd
    n = accel_amd.device_count()
    if n == 0:
        pytest.fail("no HIP device visible; gpu tests need a gfx950 GPU")
    d = accel_amd.Device(0)
    yield d


@pytest.fixture
def rng():
    return np.random.default_rng(12345)


def rel_l2(got, want) -> float:
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    den = np.linalg.norm(want)
    return float(np.linalg.norm(got - want) / (den if den > 0 else 1.0))
