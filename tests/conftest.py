import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and the built HIP library")


@pytest.fixture(scope="session")
def gpu():
    """The ROCm device; the HIP library must load (no fallback)."""
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU visible")
    from solort_amd import _lib

    _lib.load()
    return torch.device("cuda:0")
