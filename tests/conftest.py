import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


@pytest.fixture(scope="session")
def gpu():
    """The HIP device; GPU tests fail (not skip) when the device or library is missing."""
    import torch

    from dmad_amd import _native

    assert torch.cuda.is_available(), "GPU test run without a visible GPU"
    _native.lib()  # raises if libdmad_attn.so is not built
    return torch.device("cuda:0")
