import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels through the C ABI)")


@pytest.fixture(scope="session")
def gpu():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU visible (GPU tests run on the MI355X box)")
    return torch.device("cuda:0")


def pytest_collection_modifyitems(config, items):
    """The C++ driver tests start child processes that make cooperative launches; the runtime refuses
    those once this process has made its own, so that module runs before every other GPU test."""
    first = [it for it in items if it.nodeid.startswith("tests/test_gpu_cabi_driver.py")]
    if first:
        rest = [it for it in items if it not in first]
        items[:] = first + rest
