"""Shared test setup: import paths, the ``gpu`` marker, the CPU fake backend."""

import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "autokernel-halo-strix_amd")
for p in (PKG, ROOT):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


def has_gpu() -> bool:
    import torch
    return torch.cuda.is_available()


@pytest.fixture
def fake_backend(monkeypatch):
    """Route the tensor-level launchers of ``kernels.hip._lib`` to the CPU oracle."""
    import fake_backend as fb
    fb.install(monkeypatch)
    return fb
