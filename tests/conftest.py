import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
TESTS = os.path.dirname(os.path.abspath(__file__))
for p in (ROOT, TESTS):
    if p not in sys.path:
        sys.path.insert(0, p)


# Load libditch_hip.so before any test module imports torch, so that it binds
# the ROCm installation's HIP runtime (the one it is built against) rather
# than the copy inside the torch wheel, which has the same soname.
try:
    import ditch_amd

    ditch_amd.load_library()
except Exception:  # not built: the ABI tests report it
    pass


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
