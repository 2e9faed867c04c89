import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP) device and the built libpsgdk.so")


@pytest.fixture(scope="session")
def hip():
    """The loaded library; GPU tests fail loudly (not skip) when it is missing."""
    import torch
    assert torch.cuda.is_available(), "GPU test run without a visible GPU"
    from psgd_pro_amd import _lib
    return _lib.lib()
