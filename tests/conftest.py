import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) HIP device")


@pytest.fixture(scope="session")
def orc():
    import oracle

    oracle.lib()
    return oracle


@pytest.fixture(scope="session")
def dev():
    """cuda:0 for GPU tests: fails (never skips) when no device is visible, so
    a GPU run cannot pass without the HIP kernels having executed."""
    import torch

    if not torch.cuda.is_available():
        pytest.fail("no HIP device visible to torch")
    import higgs_amd

    higgs_amd.lib()
    return torch.device("cuda:0")
