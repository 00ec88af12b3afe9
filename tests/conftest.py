import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built libkvrecall.so")


@pytest.fixture(scope="session")
def ctx():
    """One kvr_context on cuda:0 for the GPU tests.  Fails (never skips)
    when the native library is missing: the HIP path is the only path."""
    import torch
    import kvmem_amd

    assert torch.cuda.is_available(), "GPU test selected but no GPU is visible"
    c = kvmem_amd.Context(0)
    yield c
    c.close()
