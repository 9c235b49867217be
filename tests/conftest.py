import sys
from pathlib import Path

import pytest
import torch

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and the built libsaeflow_hip.so")


@pytest.fixture
def device():
    return "cuda"


@pytest.fixture(autouse=True)
def _seed():
    torch.manual_seed(0)
