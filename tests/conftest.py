"""Shared pytest configuration: the `gpu` marker, repo-root imports and small helpers."""
from __future__ import annotations

import glob
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GOLDEN = os.path.join(ROOT, "tests", "golden")
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built libqvx.so")


def golden(pattern: str):
    """Sorted fixture paths under tests/golden matching pattern."""
    return sorted(glob.glob(os.path.join(GOLDEN, pattern)))


def load_npz(path: str) -> dict:
    with np.load(path, allow_pickle=False) as d:
        return {k: d[k] for k in d.files}


def max_rel(y, ref) -> float:
    """The reference's parity metric: max_i |y - ref| / max_i |ref| (cuda_backend.cu:766-772)."""
    y = np.asarray(y, np.float64)
    ref = np.asarray(ref, np.float64)
    den = max(float(np.abs(ref).max()), 1e-30) if ref.size else 1.0
    return float(np.abs(y - ref).max()) / den if ref.size else 0.0


@pytest.fixture(scope="session")
def cuda():
    """torch with a visible GPU; GPU tests fail loudly (not skip) without one."""
    import torch
    assert torch.cuda.is_available(), "GPU test run without a visible GPU"
    return torch
