"""Shared pytest setup: import paths, the `gpu` marker, device fixtures."""
from __future__ import annotations

import sys
from pathlib import Path

import pytest
import torch

REPO = Path(__file__).resolve().parent.parent
PKG_ROOT = REPO / "mini-kvllm_amd"
for p in (str(PKG_ROOT), str(REPO)):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and the built libmkv.so")


@pytest.fixture(scope="session")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU visible")
    from mkv import _lib

    _lib.load()  # raise now (not skip) if the native library is missing
    return torch.device("cuda:0")


def announce(msg: str) -> None:
    """Name the GPU case on stdout before it runs (flushed), so a run that
    dies inside a kernel still says which case it was."""
    print(f"[case] {msg}", flush=True)
