import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built libloractl_rocm.so")


@pytest.fixture(scope="session")
def cuda():
    """The GPU device; a gpu-marked test without a GPU is an error, not a skip."""
    import torch

    if not torch.cuda.is_available():
        raise RuntimeError("gpu test selected but no GPU is visible")
    torch.cuda.set_device(0)
    return torch.device("cuda:0")
