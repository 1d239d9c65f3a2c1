import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through the HIP C-ABI)")


@pytest.fixture(scope="session")
def orc():
    from oracle import oracle
    return oracle


@pytest.fixture(scope="session")
def dev():
    """The GPU under test; a GPU test without one fails rather than skips."""
    import torch
    assert torch.cuda.is_available(), "gpu-marked test needs a GPU"
    import reimagined_amd
    reimagined_amd.lib()
    return torch.device("cuda:0")
