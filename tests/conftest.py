import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs on the GPU box only)")
    config.addinivalue_line("markers", "slow: longer CPU/GPU parity runs")


@pytest.fixture(scope="session")
def oracle():
    """The CPU oracle library (built from oracle/ if missing)."""
    from tests.oracle_lib import load_oracle

    return load_oracle()


@pytest.fixture(scope="session")
def hiplib():
    """The HIP product library; fails loudly when it is not built."""
    from volta_amd import load_hip

    return load_hip()


@pytest.fixture(scope="module", autouse=True)
def subnormals_survive():
    """No library a test module loads may switch the process to
    flush-to-zero / denormals-are-zero (a -ffast-math link does that through
    crtfastmath): the oracle's subnormal arithmetic would silently change
    for every module collected after it."""
    import numpy as np

    yield
    tiny = np.float32(1e-45)  # the smallest fp32 subnormal
    assert tiny * np.float32(1.0) != 0, "denormals-are-zero is on in this process"
    assert np.float32(1.1754944e-38) / np.float32(4.0) != 0, "flush-to-zero is on in this process"
