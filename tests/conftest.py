"""Shared pytest setup: markers, paths and library handles.

`-m "not gpu"` runs the oracle against the golden vectors, the host-side logic
and the C-ABI export check; `-m gpu` runs the HIP parity tests, which call the
product library through its C ABI and compare with the oracle.
"""
from __future__ import annotations

import ctypes
import json
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
PKG = ROOT / "xks-vectorforge_amd"
GOLDEN = Path(__file__).resolve().parent / "golden"
sys.path.insert(0, str(PKG))
sys.path.insert(0, str(Path(__file__).resolve().parent))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device); run with -m gpu")


def _gpu_available() -> bool:
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


def pytest_collection_modifyitems(config, items):
    if _gpu_available():
        return
    skip = pytest.mark.skip(reason="no HIP device in this container")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(scope="session")
def oracle():
    from oracle_lib import Oracle
    return Oracle()


@pytest.fixture(scope="session")
def golden_cases():
    return json.loads((GOLDEN / "codec_cases.json").read_text())["cases"]


@pytest.fixture(scope="session")
def corruption_matrix():
    return json.loads((GOLDEN / "corruptions.json").read_text())["bases"]


@pytest.fixture(scope="session")
def hip():
    """The product library (libxksv_hip.so) through its C ABI."""
    import xksv_hip
    return xksv_hip.Library()


@pytest.fixture(scope="session")
def rng():
    return np.random.default_rng(1234)
