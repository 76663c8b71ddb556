import os
import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parent.parent
for p in (REPO, REPO / "pytorch-xdna2_amd"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (run on the GPU box with -m gpu)")
    config.addinivalue_line("markers", "slow: long CPU oracle runs")


@pytest.fixture(scope="session")
def hip():
    """The C-ABI library; GPU tests fail (not skip) when it or the GPU is missing."""
    import torch
    from xdna_train import hip_abi

    lib = hip_abi.load()
    assert torch.cuda.is_available(), "GPU test run without a visible GPU"
    torch.cuda.init()
    return lib


@pytest.fixture
def stream():
    import torch

    return torch.cuda.current_stream().cuda_stream
