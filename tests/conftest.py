import importlib
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP device (MI355X); runs through libetmoe.so")


@pytest.fixture(scope="session")
def orc():
    """The CPU oracle (test infrastructure), built on first use."""
    import oracle
    oracle.build()
    return oracle


@pytest.fixture(scope="session")
def et():
    """The product package (imports torch, loads libetmoe.so lazily)."""
    return importlib.import_module("peer-review-agents_amd")


@pytest.fixture(scope="session")
def dev():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no HIP device in this environment")
    return torch.device("cuda:0")
