"""Shared test configuration: markers, seeded inputs and the parity metric."""

from __future__ import annotations

import math
import os
import sys

import numpy as np
import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


def rel_l2(got_re, got_im, ref_re, ref_im) -> float:
    """||got - ref||_2 / ||ref||_2 over both planes (float64 accumulation)."""
    def f64(t):
        if isinstance(t, torch.Tensor):
            t = t.detach().cpu().numpy()
        return np.asarray(t, dtype=np.float64)

    gr, gi, rr, ri = f64(got_re), f64(got_im), f64(ref_re), f64(ref_im)
    num = np.sqrt(((gr - rr) ** 2).sum() + ((gi - ri) ** 2).sum())
    den = np.sqrt((rr**2).sum() + (ri**2).sum())
    return float(num / den) if den > 0 else float(num)


def tol_pow2(n: int) -> float:
    """fp32 parity bound for power-of-two transforms: 1e-6 * log2(n)."""
    return 1e-6 * max(1.0, math.log2(n))


def tol_bluestein(n: int) -> float:
    """fp32 parity bound for Bluestein transforms: 1e-5 * log2(n)."""
    return 1e-5 * max(1.0, math.log2(n))


def seeded_complex(batch: int, n: int, seed: int = 42):
    """re then im ~ N(0,1) from one generator (reference tests/conftest.py:52-55)."""
    g = torch.Generator().manual_seed(seed)
    re = torch.randn(batch, n, generator=g)
    im = torch.randn(batch, n, generator=g)
    return re, im


@pytest.fixture
def rng():
    return torch.Generator().manual_seed(42)
