import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
TESTS = os.path.dirname(os.path.abspath(__file__))
for p in (ROOT, TESTS):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP library)")


@pytest.fixture(scope="session")
def ref():
    from oracle.ref import Ref
    return Ref()


@pytest.fixture(scope="session")
def dev():
    from ditch_amd.hip import Device
    d = Device(0)
    yield d
    d.close()
