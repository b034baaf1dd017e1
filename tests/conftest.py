import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)
TESTS = os.path.dirname(os.path.abspath(__file__))
if TESTS not in sys.path:
    sys.path.insert(0, TESTS)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) device; runs the HIP backend")


@pytest.fixture(scope="session")
def plane():
    """The device context. On a GPU run a missing device or library is an error, not a skip."""
    from bramha_amd.plane import HipComputePlane

    p = HipComputePlane(0)
    yield p
    p.close()
