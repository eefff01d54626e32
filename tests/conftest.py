import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and the built HIP library")


@pytest.fixture(scope="session")
def gpu_device():
    """The GPU tests' device; fails (not skips) when there is no GPU or library."""
    import torch

    from pagelora_amd import _lib

    assert torch.cuda.is_available(), "GPU test run without a visible ROCm GPU"
    _lib.load()
    return torch.device("cuda:0")
