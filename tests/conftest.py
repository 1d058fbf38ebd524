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
