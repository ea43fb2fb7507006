import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a real MI355X (runs through the C ABI)")


@pytest.fixture(scope="session")
def dev():
    """One HIP device for the whole GPU session (tests run in one process)."""
    from sanic_amd.backend import HipDevice
    d = HipDevice(0)
    yield d
