"""Shared test setup: the `gpu` marker, the oracle CPU device and helpers."""
from __future__ import annotations

import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device)")


@pytest.fixture(scope="session")
def fg():
    import ferrograd_amd

    ferrograd_amd.lib()
    return ferrograd_amd


@pytest.fixture(scope="session")
def cpu(fg):
    """Registers the oracle's CPU device ("cpu") and returns its device name."""
    import oracle

    oracle.load()
    return "cpu"


@pytest.fixture(scope="session")
def hip(fg):
    """The HIP device name; fails loudly when the native HIP path is unusable."""
    import torch  # noqa: F401  (only to report availability clearly)

    return "hip"


def seeded(seed: int):
    return np.random.default_rng(seed)


def rel_err_bound(got: np.ndarray, want: np.ndarray, scale: np.ndarray, tol: float) -> float:
    """max |got-want| / (tol * scale) — <= 1 passes (scale = sum |terms|)."""
    denom = np.maximum(scale.astype(np.float64), np.finfo(np.float32).tiny) * tol
    return float(np.max(np.abs(got.astype(np.float64) - want.astype(np.float64)) / denom))
