import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and the built libtlx_hip.so")


@pytest.fixture(scope="session")
def gpu():
    """The GPU parity tests run only where a GPU exists; there they must find the HIP library
    (no fallback)."""
    import torch
    assert torch.cuda.is_available(), "GPU test collected on a machine without a GPU"
    from thunderllamax_amd import _lib
    _lib.lib()
    return torch.device("cuda:0")
