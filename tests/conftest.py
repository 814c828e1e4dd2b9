import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(REPO, "dryft-challenge_amd")
for p in (PKG, REPO):
    if p not in sys.path:
        sys.path.insert(0, p)

os.environ.setdefault("USE_HUB_KERNELS", "0")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through libqdec.so)")


def gpu_available():
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


@pytest.fixture(scope="session")
def qlib():
    from qdec import capi
    return capi.lib()
