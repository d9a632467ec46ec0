"""GEMV activations outside N(0,1): outlier channels and non-finite values.

The integer GEMV kernels convert each 64-element slot of x to 15-bit fixed point scaled by the slot's
largest |x|, so an element's conversion error scales with that maximum (<= 3.1e-5 of it).  LLM hidden
states carry outlier channels of 100-1000x the typical magnitude; with one such outlier in every slot
the small elements lose most of their bits, but the sum is dominated by the outliers and the error
stays inside the GEMV bar (1e-3 max-relative against the exact fp64 sum, the reference's metric,
cuda_backend.cu:766-772).  Checked for every fast GEMV family at M = 1 and batched (bit-identity
across batch sizes is tested elsewhere).

Non-finite activations: the reference's fp32 dot products (qmatmul.cpp:28-62) turn a row into +-Inf,
or NaN where a zero weight meets Inf or +Inf meets -Inf.  The engine's converted slot holds NaN once
its maximum is infinite, so every output reading that slot is NaN.  The contract tested here: an
output is non-finite exactly where the reference's is (the kind, Inf or NaN, may differ), and NaN
inputs give NaN outputs in both.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
import qorvix_amd as qvx
from conftest import max_rel
from test_gpu_kernels import random_weight, run_gemv

pytestmark = pytest.mark.gpu

GEMV_TOL = 1e-3
FAMILIES = [(qvx.Q4_K, 1024, 4096), (qvx.Q4_K, 512, 14336), (qvx.Q6_K, 1024, 4096), (qvx.Q8_0, 512, 4096),
            (qvx.Q4_0, 512, 4096), (qvx.Q5_K, 512, 4096), (qvx.Q5_0, 512, 4096)]


def _outlier_x(rng, nvec, cols, scale):
    x = rng.standard_normal((nvec, cols)).astype(np.float32)
    slots = cols // 64
    pos = rng.integers(0, 64, size=(nvec, slots)) + 64 * np.arange(slots)[None, :]
    sign = rng.choice([-1.0, 1.0], size=(nvec, slots))
    for v in range(nvec):
        x[v, pos[v]] = (sign[v] * scale * (1.0 + rng.random(slots))).astype(np.float32)
    return x


@pytest.mark.parametrize("t,rows,cols", FAMILIES)
@pytest.mark.parametrize("scale", [100.0, 1000.0])
@pytest.mark.parametrize("nvec", [1, 8])
def test_gemv_outlier_channels_within_bar(cuda, t, rows, cols, scale, nvec):
    rng = np.random.default_rng(int(scale) + rows + cols + t + nvec)
    w = random_weight(t, rows, cols, rng, scale=0.002)
    X = _outlier_x(rng, nvec, cols, scale)
    got = run_gemv(cuda, w, t, X, rows, cols)
    ref = oracle.matmul_f64(w, t, X, nvec, rows, cols)
    assert np.isfinite(got).all()
    for v in range(nvec):
        assert max_rel(got[v], ref[v]) <= GEMV_TOL, v


@pytest.mark.parametrize("t,rows,cols", FAMILIES)
def test_gemv_non_finite_activations(cuda, t, rows, cols):
    rng = np.random.default_rng(rows + cols + t)
    w = random_weight(t, rows, cols, rng, scale=0.002)
    X = rng.standard_normal((4, cols)).astype(np.float32)
    X[0, 70] = np.inf            # one +Inf
    X[1, 3] = -np.inf            # one -Inf in another slot
    X[1, cols - 1] = np.inf      # ... and a +Inf: rows may see Inf - Inf
    X[2, 200] = np.nan           # NaN
    # X[3] stays finite
    got = run_gemv(cuda, w, t, X, rows, cols)
    for v in range(4):
        ref = oracle.qmatmul(w, t, X[v], rows, cols)
        np.testing.assert_array_equal(np.isfinite(got[v]), np.isfinite(ref), err_msg=f"vector {v}")
        np.testing.assert_array_equal(np.isnan(got[v]) | np.isfinite(got[v]), np.ones(rows, bool))
    assert np.isnan(got[2]).all()
    assert np.isfinite(got[3]).all()
    ref3 = oracle.matmul_f64(w, t, X[3:4], 1, rows, cols)
    assert max_rel(got[3:4], ref3) <= GEMV_TOL
