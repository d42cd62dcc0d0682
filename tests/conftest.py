import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "glm-flash-rs_amd")
for p in (PKG, os.path.join(ROOT, "oracle"), ROOT):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and the built libgfr_moe.so")


@pytest.fixture(scope="session")
def oracle():
    import oracle as o
    o.lib()
    return o


@pytest.fixture(scope="session")
def gfr():
    """The HIP library; GPU tests fail loudly (no fallback) when it or the GPU is missing."""
    import torch
    import gfr_moe
    assert torch.cuda.is_available(), "GPU test without a GPU"
    gfr_moe.lib()
    return gfr_moe
