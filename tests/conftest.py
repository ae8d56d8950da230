"""Shared fixtures.  GPU tests are marked `gpu`; everything else runs on CPU."""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through libglypr_hip.so)")


@pytest.fixture(scope="session")
def oracle():
    from oracle import pyoracle
    pyoracle.lib()
    return pyoracle


@pytest.fixture(scope="session")
def ctx():
    """A glypr_hip context on cuda:0.  GPU tests fail (not skip) without a GPU."""
    import torch
    from glypr_amd.ops import Context
    assert torch.cuda.is_available(), "GPU test run without a visible GPU"
    c = Context(0)
    yield c
    torch.cuda.synchronize()
    c.close()
