"""Shared test setup: import paths, the `gpu` marker, seeded input generators."""
from __future__ import annotations

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
PKG_PARENT = ROOT / "specdec-context-scaling_amd"
for p in (str(ROOT), str(PKG_PARENT)):
    if p not in sys.path:
        sys.path.insert(0, p)

GOLDEN = ROOT / "tests" / "golden"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built libsdv.so")


@pytest.fixture(scope="session")
def cuda_device():
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU test selected but no HIP device is visible")
    from specdec_amd import _native

    _native.load()  # fail loudly if the native library was not built
    return torch.device("cuda:0")


def announce(msg: str) -> None:
    """Name the case before a GPU step (flushed, so a fault still leaves the name behind)."""
    print(f"[case] {msg}", flush=True)
