"""pytest configuration: markers and shared fixtures.

`-m "not gpu"` runs the oracle checks, host logic and ABI checks (no device);
`-m gpu` runs the parity tests of the gfx950 kernels through the C-ABI.
"""
import os
import sys

import pytest

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))

import _util  # noqa: E402


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP device (MI355X / gfx950)")


@pytest.fixture(scope="session")
def lib():
    return _util.load_lib()


@pytest.fixture(scope="session")
def orc():
    return _util.load_oracle()


@pytest.fixture(scope="session")
def ref():
    r = _util.load_ref()
    if r is None:
        pytest.skip("oracle/_ref (reference sources) not built here")
    return r


@pytest.fixture(scope="session")
def dev():
    """torch device for GPU tests; the library must see the same device."""
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    return torch.device("cuda:0")
