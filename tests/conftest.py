import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through the HIP library)")


@pytest.fixture(scope="session")
def gpu():
    """The CUDA (HIP) device; fails loudly if the GPU or the native library is missing."""
    import torch

    assert torch.cuda.is_available(), "GPU test on a machine without a GPU"
    from kvskip_amd import _native

    _native.lib()
    return torch.device("cuda:0")
