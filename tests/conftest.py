import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


@pytest.fixture(scope="session")
def oracle():
    import oracle as o

    o.lib()
    return o


@pytest.fixture(scope="session")
def gpu():
    """The GPU test fixture: fails (never skips) when the device or the
    native library is missing, so a GPU run cannot pass on a fallback."""
    import torch

    assert torch.cuda.is_available(), "GPU tests need a ROCm device"
    from tcc_amd import _lib

    _lib.lib()
    return torch.device("cuda:0")
