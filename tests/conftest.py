import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "exllamav3-rs_amd"), os.path.join(ROOT, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (run with -m gpu on the GPU box)")


@pytest.fixture(autouse=True)
def _faithful_oracle():
    """Every test starts and ends with the oracle's planted-mistake switch off."""
    from oracle import oracle as orc
    orc.set_mutation(0)
    yield
    orc.set_mutation(0)


@pytest.fixture(scope="session")
def cuda():
    import torch
    assert torch.cuda.is_available(), "GPU test run without a GPU"
    return torch.device("cuda:0")
