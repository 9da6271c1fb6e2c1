import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through libtensorium_hip on cuda:0)")
    config.addinivalue_line("markers", "slow: large shapes")


@pytest.fixture(scope="session")
def hip():
    """The TNNHip backend object on device 0 (GPU tests only)."""
    import torch

    from tensorium_amd.nnhip import TNNHip

    assert torch.cuda.is_available(), "GPU test collected without a GPU"
    h = TNNHip(0)
    h.useTorchStream()  # order library kernels with torch's allocations/copies
    yield h
    h.finish()


@pytest.fixture(scope="session")
def dev():
    import torch

    return torch.device("cuda:0")
