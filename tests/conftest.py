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


@pytest.fixture(params=[-1, 0, 1, 2, 3, 4], ids=["cfg_auto", "cfg256x8", "cfg128x4", "cfg256x4", "cfg256ws",
                                                   "cfg128ws"])
def b16cfg(request, hip):
    """Forces the bf16 kernel's tile configuration (-1: chosen by size; 0: 256 x 256 tiles on 8 waves, the
    ping-pong main loop; 1: 128 x 128 on 4 waves; 2: 256 x 256 on 4 waves; 3: 256 x 256 on 8 MFMA waves and 4
    producer waves, the warp-specialized main loop; 4: 128 x 128 on 4 MFMA waves and 4 producer waves) for one
    test, then restores it."""
    assert hip.psgdk_set_option(1, request.param) == 0
    yield request.param
    hip.psgdk_set_option(1, -1)
