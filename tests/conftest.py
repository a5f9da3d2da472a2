import importlib
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP device (MI355X)")


def load_gi():
    """The product package (directory name go-infer_amd)."""
    return importlib.import_module("go-infer_amd")


@pytest.fixture(scope="session")
def gi():
    return load_gi()


@pytest.fixture(scope="session")
def oracle():
    import oracle as o
    o.lib()
    return o


@pytest.fixture(scope="session")
def dev():
    """cuda:0 with the HIP library loaded; GPU tests fail loudly if either
    is missing (no CPU fallback exists)."""
    import torch
    assert torch.cuda.is_available(), "GPU test run without a HIP device"
    g = load_gi()
    g.lib()
    return torch.device("cuda:0")
