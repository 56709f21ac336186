import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built libhwk")
    config.addinivalue_line("markers", "slow: a long GPU case (full model sizes)")


@pytest.fixture(scope="session")
def orc():
    from oracle import oracle

    oracle.lib()
    return oracle


@pytest.fixture(scope="session")
def dev():
    """cuda:0 with libhwk loaded; the GPU tests need both (no CPU fallback to test)."""
    import torch

    from hwnpu_amd import hwk

    if not torch.cuda.is_available():
        pytest.fail("GPU test without a GPU")
    hwk.load()
    torch.cuda.init()
    return torch.device("cuda:0")
