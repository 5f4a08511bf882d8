import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and libnerve_hip.so")


@pytest.fixture(scope="session")
def ctx():
    """One nerve_hip context for the whole GPU session (device 0)."""
    import torch
    from nerve_amd.hip import Context

    assert torch.cuda.is_available(), "GPU tests need a visible GPU"
    c = Context(0)
    yield c
    torch.cuda.synchronize()
    c.close()


@pytest.fixture(scope="session")
def dev():
    import torch

    return torch.device("cuda:0")
