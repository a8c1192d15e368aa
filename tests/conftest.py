import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)
HERE = os.path.dirname(os.path.abspath(__file__))
if HERE not in sys.path:
    sys.path.insert(0, HERE)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through libhip_bridge.so)")


@pytest.fixture(scope="session")
def oracle():
    from oracle import oracle as O
    return O.get()


@pytest.fixture(scope="session")
def dev():
    from ziglm_amd.device import HipDevice
    d = HipDevice()
    yield d
    d.sync()
