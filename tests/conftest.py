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
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; runs the HIP kernels")


@pytest.fixture(scope="session")
def cuda():
    """The GPU device (fails, not skips, when a gpu-marked test runs without one)."""
    import torch

    if not torch.cuda.is_available():
        pytest.fail("gpu test run without a GPU")
    torch.cuda.init()
    return torch.device("cuda:0")
