"""Shared fixtures.  ``gpu`` marks tests that need an MI355X and the built
HIP library; everything else runs on the CPU."""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a GPU and libzorse_amd.so")


@pytest.fixture(scope="session")
def dev():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from zorse_amd import _abi
    _abi.lib()  # raises if the library is missing: GPU tests never run without it
    return torch.device("cuda:0")
