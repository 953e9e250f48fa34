import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP GPU (MI355X); run with -m gpu")


@pytest.fixture(scope="session")
def kdecay_lib():
    """libkdecay.so, built in-tree if it is not there yet."""
    from kilat_amd import _build, _lib

    if not os.path.exists(_build.LIBRARY):
        _build.build_library()
    return _lib.load()


@pytest.fixture(scope="session")
def hip_device():
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU test selected but no HIP device is visible")
    return torch.device("cuda", 0)
