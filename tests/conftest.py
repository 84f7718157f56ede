import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

import __graft_entry__  # noqa: E402

PKG = __graft_entry__.load_package()


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built library")


def gpu_available() -> bool:
    import torch
    return torch.cuda.is_available()


@pytest.fixture(scope="session")
def pkg():
    return PKG


@pytest.fixture(scope="session")
def wl():
    from importlib import import_module
    return import_module("fni8serve_amd.workloads")


@pytest.fixture(scope="session")
def cuda():
    """GPU tests fail (not skip) without a GPU: a silent skip would hide that the
    HIP path never ran."""
    import torch
    if not torch.cuda.is_available():
        pytest.fail("GPU test run without a visible GPU")
    return torch.device("cuda:0")
