"""Shared test setup: the `gpu` marker, import paths, and the GPU-side fixtures."""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; run with -m gpu")


@pytest.fixture(scope="session")
def torch_dev():
    """torch on the GPU, used only for device buffers and streams."""
    import torch

    if not torch.cuda.is_available():
        pytest.fail("a gpu test ran on a host without a GPU")
    return torch


@pytest.fixture(scope="session")
def hip_backend():
    from tritify_amd import HipBackend

    b = HipBackend(0)
    yield b
    b.close()
