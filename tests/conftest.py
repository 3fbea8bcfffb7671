import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) device")


@pytest.fixture(scope="session")
def oracle():
    import oracle as o
    o.build()
    return o


@pytest.fixture(scope="session")
def dev():
    """The HIP backend on cuda:0.  GPU tests fail (not skip) without it: they
    are only selected with -m gpu, on a GPU box."""
    import torch
    import momijo_amd
    from momijo_amd import _lib
    assert torch.cuda.is_available(), "no GPU visible to torch"
    assert _lib.device_available(), "libmomijo_hip reports no gfx950 device"
    torch.cuda.set_device(0)
    return torch.device("cuda", 0)
