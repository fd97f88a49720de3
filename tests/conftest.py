"""Shared test setup: the `gpu` marker, import paths, device fixtures."""

import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "flashengine.cpp_amd")
for p in (ROOT, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a real MI355X (HIP device) and the built library")


@pytest.fixture(scope="session")
def dev():
    """The HIP device; GPU tests fail (not skip) when the library is missing."""
    import torch

    import feattn

    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    feattn.lib()  # raises if libfeattn.so is not built: no silent fallback
    torch.cuda.set_device(0)
    return torch.device("cuda", 0)
