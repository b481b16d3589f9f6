import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X); parity of the HIP kernels against the oracle")


def gpu_available() -> bool:
    import torch

    return torch.cuda.is_available() and torch.version.hip is not None


@pytest.fixture(scope="session")
def device():
    import torch

    if not gpu_available():
        pytest.skip("no ROCm GPU")
    return torch.device("cuda:0")
