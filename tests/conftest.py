import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG_ROOT = os.path.join(ROOT, "triton-ext_amd")
for p in (ROOT, PKG_ROOT):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def gpu():
    """Skip unless a gfx950 device is visible; then the HIP extension must load."""
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import triton_ext_amd as tx
    L = tx.load()  # raises if libmi355x_dot.so is missing: no fallback
    if not L.tx_device_available():
        pytest.skip("GPU is not gfx950")
    return torch.device("cuda:0")
