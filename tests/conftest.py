import importlib
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


@pytest.fixture(scope="session")
def qmv():
    """The package under test (directory name is not an identifier)."""
    return importlib.import_module("my-inference-engine_amd")


@pytest.fixture(scope="session")
def oracle():
    import oracle as o
    o.lib()  # raises if liboracle.so was not built
    return o


@pytest.fixture(scope="session")
def gpu(qmv):
    """Skip-free GPU gate: a gpu-marked test must find a device."""
    n = qmv.hip_lib().qmv_device_count()
    assert n > 0, "no HIP device visible"
    return n
