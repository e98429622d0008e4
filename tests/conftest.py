import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for path in (ROOT, os.path.join(ROOT, "oracle")):
    if path not in sys.path:
        sys.path.insert(0, path)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs on the GPU box)")
    config.addinivalue_line("markers", "slow: long-running parity case")


@pytest.fixture(scope="session")
def oracle():
    import oracle as o  # oracle/oracle.py
    o.lib()
    return o


@pytest.fixture(scope="session")
def device():
    from dolittle_amd import Device
    return Device(0)


@pytest.fixture(scope="session")
def queue(device):
    return device.create_queue()
