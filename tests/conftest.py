"""Shared test setup.

CPU tests (default, `-m "not gpu"`): oracle pinning against the reference's
golden vectors, host-side logic, and the C ABI's exports.
GPU tests (`-m gpu`): parity of the HIP path (through the C ABI) with the
oracle and the golden fixtures; they fail, never skip, when no GPU is visible.
"""
from __future__ import annotations

import json
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
GOLDEN = ROOT / "tests" / "golden"
sys.path.insert(0, str(ROOT / "minimind-orangepi_amd"))
sys.path.insert(0, str(ROOT / "oracle"))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


def load_golden(name: str) -> dict:
    data = json.loads((GOLDEN / f"{name}.json").read_text())
    path = GOLDEN / f"{name}_logits.npy"
    data["logits"] = np.load(path) if path.exists() else None
    return data


def rel_err(a, b) -> float:
    """max |a - b| / max |b|: the normwise relative error used for every
    floating-point parity check (tolerance 2e-3 for logits / attention)."""
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    denom = max(float(np.max(np.abs(b))), 1e-30)
    return float(np.max(np.abs(a - b))) / denom


@pytest.fixture(scope="session")
def mmr():
    import mmr as m  # noqa: WPS433

    return m


@pytest.fixture(scope="session")
def oracle():
    import oracle as o  # noqa: WPS433

    return o


@pytest.fixture(scope="session")
def gpu(mmr):
    if mmr.device_count() < 1:
        pytest.fail("no HIP device visible: GPU tests must run on the MI355X box")
    return mmr
