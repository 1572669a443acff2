import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for path in (ROOT, os.path.join(ROOT, "tests")):
    if path not in sys.path:
        sys.path.insert(0, path)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a gfx950 GPU (MI355X); runs the HIP kernels")


@pytest.fixture(scope="session")
def context():
    """One HIP context for the GPU tests of a session (device 0)."""
    import satori_amd

    ctx = satori_amd.HipContext(0)
    yield ctx
