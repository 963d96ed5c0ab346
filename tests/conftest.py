"""Shared test setup: import paths, the ``gpu`` marker, and GPU fixtures."""

from __future__ import annotations

import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
PKG_PARENT = ROOT / "strix-halo-int4-gemms_amd"
for p in (str(PKG_PARENT), str(ROOT)):
    if p not in sys.path:
        sys.path.insert(0, p)

os.environ.setdefault("OMP_NUM_THREADS", str(min(16, os.cpu_count() or 1)))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a gfx950 GPU and the built kernel library")


@pytest.fixture(scope="session")
def device():
    """The GPU every gpu-marked test runs on.  Fails (never skips) when the GPU
    or the kernel library is missing, so a GPU run cannot pass silently."""
    import torch

    assert torch.cuda.is_available(), "gpu tests need a ROCm GPU"
    from amd_strix_halo_kernels import native

    status = native.dispatch_runtime_status()
    assert status.has_linked_kernels, f"no gfx950 device for the linked kernels: {status}"
    return torch.device("cuda:0")
