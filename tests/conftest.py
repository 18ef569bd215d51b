import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "flash-evict-prefill_amd")
for p in (PKG, ROOT):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP GPU (MI355X) and the built library")


@pytest.fixture(autouse=True)
def _precision():
    import torch
    torch.manual_seed(731)
    torch.backends.cuda.matmul.allow_tf32 = False
    yield
