"""Shared test setup: import paths, the `gpu` marker, device helpers."""

from __future__ import annotations

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
PKG = ROOT / "luciole-1b_amd"
for p in (str(ROOT), str(PKG)):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU and the built HIP library")


@pytest.fixture(scope="session")
def gpu():
    """The CUDA (HIP) device; skips when no GPU is visible, fails if the library is missing."""
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    from SSA import _lib

    _lib.lib()  # raises when libssa_mi355x.so was not built: no silent fallback
    return torch.device("cuda:0")
