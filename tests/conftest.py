import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP device (MI355X); the parity tests proper")


@pytest.fixture(scope="session")
def dev():
    from vernondsl_amd import rhi
    n = rhi.device_count()
    if n < 1:
        pytest.fail("GPU test run without a HIP device (run with -m 'not gpu' on a CPU host)")
    d = rhi.Device(0)
    yield d


@pytest.fixture(scope="session")
def q(dev):
    from vernondsl_amd import rhi
    queue = rhi.Queue(dev)
    yield queue
