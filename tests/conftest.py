"""Shared pytest setup: the `gpu` marker, repo-root imports and the package fixture."""

from __future__ import annotations

import importlib
import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parents[1]
if str(REPO) not in sys.path:
    sys.path.insert(0, str(REPO))

PACKAGE_NAME = "gpu-kernel-for-transformer_amd"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built libxblock.so")


@pytest.fixture(scope="session")
def pkg():
    return importlib.import_module(PACKAGE_NAME)


@pytest.fixture(scope="session")
def capi():
    return importlib.import_module(PACKAGE_NAME + "._capi")


@pytest.fixture(scope="session")
def cuda():
    """The GPU device; GPU tests fail (not skip) when the library or device is missing."""
    import torch

    capi = importlib.import_module(PACKAGE_NAME + "._capi")
    if not capi.XBLOCK_AVAILABLE:
        raise RuntimeError(f"libxblock.so unavailable: {capi.XBLOCK_LOAD_ERROR}")
    if not torch.cuda.is_available():
        raise RuntimeError("GPU tests need a visible MI355X")
    device = torch.device("cuda:0")
    arch = capi.gfx_arch(device)
    if arch != "gfx950":
        raise RuntimeError(f"GPU tests need gfx950, found {arch}")
    return device
