"""Shared test setup: the `gpu` marker, import paths and build checks."""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "voxcpm-cpp_amd"), os.path.join(ROOT, "oracle")):
    if p not in sys.path:
        sys.path.insert(0, p)

GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


@pytest.fixture(scope="session")
def orc():
    import oracle

    oracle.lib()
    return oracle


@pytest.fixture(scope="session")
def vxm_ctx():
    """One library context on cuda:0 for the whole GPU session."""
    import torch
    import vxm

    assert torch.cuda.is_available(), "GPU tests need a GPU"
    torch.cuda.init()
    ctx = vxm.Context(0)
    yield ctx
    ctx.close()
