import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X); runs the HIP kernels")
    config.addinivalue_line("markers", "slow: long-running CPU test")


@pytest.fixture(autouse=True)
def _device_comp_exp2(request):
    """GPU tests compare the kernels with the oracle compositing with the same
    G: the device's exp2 instruction, whose values the oracle takes from a
    table built on the first GPU test (CPU tests keep the oracle's exp2n)."""
    from tests import _util
    if request.node.get_closest_marker("gpu") is not None:
        _util.use_device_comp_exp2()
    else:
        _util.use_default_comp_exp2()
    yield


@pytest.fixture(scope="session")
def oracle():
    from oracle import pyoracle
    pyoracle.load()
    return pyoracle
