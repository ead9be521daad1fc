import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device) and the built libqws.so")


@pytest.fixture(scope="session")
def sampler():
    import torch
    import qwen_warp_amd as q
    assert torch.cuda.is_available(), "GPU test without a GPU"
    return q.Sampler("cuda")
