"""Shared pytest setup: the `gpu` marker, repo root on sys.path, GPU fixtures."""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and the built HIP library")


@pytest.fixture(scope="session")
def hip():
    """The HIP backend (loads libifkfac_hip.so); skips when no GPU is visible."""
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU visible")
    from ifkfac_amd import _backend
    be = _backend.HipBackend()
    _backend.set_backend(be)
    return be
