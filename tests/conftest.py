"""Shared fixtures.  ``gpu`` tests need an MI355X (HIP device) and the built
``gbxcule_amd/lib/libgbx_hip.so``; everything else runs on the CPU."""

from __future__ import annotations

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP GPU and libgbx_hip.so")
    config.addinivalue_line("markers", "slow: long-running CPU test")


@pytest.fixture(scope="session")
def bootstub() -> bytes:
    from gbxcule_amd.carts.bootstub import build_bootstub

    return build_bootstub()


@pytest.fixture(scope="session")
def carts() -> dict[str, bytes]:
    from gbxcule_amd.carts.synth import CARTS

    return {name: fn() for name, fn in CARTS.items()}


def require_gpu() -> None:
    try:
        import torch
    except Exception as exc:  # pragma: no cover
        pytest.skip(f"torch unavailable: {exc}")
    if not torch.cuda.is_available():
        pytest.fail("gpu test collected without a HIP device")
