import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (ROCm device) and the built HIP library")


@pytest.fixture(scope="session")
def device():
    """The GPU. GPU tests fail (they do not skip) when there is none: a GPU run
    that silently skipped would look green without having exercised the kernels."""
    import torch
    assert torch.cuda.is_available(), "gpu-marked test needs a ROCm device"
    return torch.device("cuda:0")
