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
    """The GPU device for `gpu` tests; fails loudly if the HIP path is missing."""
    import torch

    from fna2_amd import _capi

    assert torch.cuda.is_available(), "gpu test run without a GPU"
    _capi.lib()  # raises if libfna2_hip.so is missing
    return torch.device("cuda:0")
