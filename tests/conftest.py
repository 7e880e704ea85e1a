import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "mojo-gemma4-cpu_amd")
for p in (ROOT, PKG, os.path.join(ROOT, "oracle")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP library)")


@pytest.fixture(scope="session")
def O():
    import oracle
    oracle.lib()
    return oracle


@pytest.fixture(scope="session")
def gpu():
    """The HIP library on cuda:0.  A GPU test must never fall back to CPU:
    if the device or libbq.so is missing this fails loudly."""
    import torch
    assert torch.cuda.is_available(), "GPU test collected on a machine without a GPU"
    import bq
    bq.init(0)
    return bq
