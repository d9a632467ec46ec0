"""GPU parity at the BASELINE configurations' full sizes, for every kernel instantiation the bench
reports: the prefill GEMM's 256- and 128-token tiles (config 4 at M = 128 / 512 / 1024 / 1025 /
2048, the stacked 28672-row gate|up weight at M = 257), the Q6_K LM head at M = 16 and Q4_K
qmatmul_n at M = 512 (config 3 shapes).

The outputs are checked on a strided slice of weight rows (every 37th or 97th row: strides prime to
the 16 / 32 / 64 / 256-row tile and wave boundaries, so every lane position and tile is sampled) and
every token, against the oracle's exact dequantised values (oracle/qvx_oracle.c, bit-exact with the
reference's dequant.cpp) multiplied in float64.  Two bars per 16-bit GEMM variant:
  * the north star's 2e-2 max-relative against the exact product;
  * a much tighter bar against the product of the operands rounded the way the variant rounds them
    (bf16: X and W each rounded to nearest even; fp16: W rounded, X exact), where what is left is
    fp32 accumulation error plus the kernels' dequantisation: they evaluate d*sc*n - dmin*m as
    (1024 + n) * ds + (dm - 1024 ds) with the bias rounded once to fp32 (an error of up to 2^-14 ds),
    so about 2^-14 / 2^-8 of the bf16 roundings (2^-14 / 2^-11 of the fp16 ones) land one ulp from
    round-to-nearest.  Over K = 4096 random terms that is ~1e-4 of max|ref| for bf16 and ~5e-5 for
    fp16; the bars are 1e-3 and 2e-4.  A dropped or repeated 64-element K slice, a wrong scale or a
    swapped operand moves the result by ~3e-2 (sqrt(64 / K) of a typical output, a quarter of the
    largest): one to two orders of magnitude above them.
The int8 variant is held at 1e-4 against the oracle's Q8 quantisation of X times the exact weights.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
import qorvix_amd as qvx
from conftest import max_rel

pytestmark = pytest.mark.gpu

GEMM_TOL = 2e-2        # north star, 16-bit MFMA path
ROUNDED_TOL = {0: 1e-3, 2: 2e-4}  # against the variant's own operand rounding (bf16, fp16)
I8_TOL = 1e-4          # int8 variant against the Q8-quantised oracle
GEMV_TOL = 1e-3


def _bf16_round(a32: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 (round to nearest even), returned as fp64 (finite inputs)."""
    u = np.ascontiguousarray(a32, np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint32) << 16
    return r.view(np.float32).astype(np.float64)


def _row_slice(w_bytes: np.ndarray, t: int, rows: int, cols: int, idx: np.ndarray) -> np.ndarray:
    """Exact fp32 dequantised values of weight rows idx, [len(idx), cols]."""
    bs, ts = qvx.type_traits(t)
    rb = cols // bs * ts
    sel = w_bytes.reshape(rows, rb)[idx].reshape(-1)
    return oracle.dequantize(t, sel, len(idx) * cols).reshape(len(idx), cols)


def _check_gemm(cuda, t, M, rows, cols, variants, seed, stride=37):
    W = qvx.empty_weight(t, rows, cols)
    qvx.fill_synthetic_t(W, t, rows, cols, seed=seed, scale_mul=1e-3)
    X = cuda.empty((M, cols), dtype=cuda.float16, device="cuda")
    qvx.fill_normal_t(X, seed=seed + 1, mul=0.5)
    cuda.cuda.synchronize()
    idx = np.arange(0, rows, stride)
    idx = np.union1d(idx, [rows - 1])
    Wd = _row_slice(W.cpu().numpy(), t, rows, cols, idx)
    X32 = X.cpu().numpy().astype(np.float32)
    exact = X32.astype(np.float64) @ Wd.astype(np.float64).T
    for variant in variants:
        out = qvx.qgemm_t(W, t, X, rows, cols, variant)
        cuda.cuda.synchronize()
        got = out.cpu().numpy()[:, idx]
        assert np.isfinite(got).all(), (M, rows, cols, variant)
        if variant == qvx.GEMM_I8:
            q, s, _ = oracle.quantize_q8_act(X32)
            Xq = q.astype(np.float64) * np.repeat(s.astype(np.float64), 32, axis=1)
            assert max_rel(got, Xq @ Wd.astype(np.float64).T) <= I8_TOL, (M, rows, cols, variant)
        else:
            assert max_rel(got, exact) <= GEMM_TOL, (M, rows, cols, variant)
            if variant == qvx.GEMM_BF16:
                rounded = _bf16_round(X32) @ _bf16_round(Wd).T
            else:
                rounded = X32.astype(np.float64) @ Wd.astype(np.float16).astype(np.float64).T
            err = max_rel(got, rounded)
            assert err <= ROUNDED_TOL[variant], (M, rows, cols, variant, err)


ALL16 = (qvx.GEMM_BF16, qvx.GEMM_F16)


@pytest.mark.parametrize("M", [2048, 1025, 1024, 512, 128])
def test_gemm_q4k_config4_full(cuda, M):
    """Config 4 (Q4_K 4096 -> 14336) at every M the bench reports and at the 256-token tile policy's
    edges (M = 1024: whole 256-token tiles; 1025: a one-token last tile), all three variants."""
    _check_gemm(cuda, qvx.Q4_K, M, 14336, 4096, ALL16 + (qvx.GEMM_I8,), seed=7000 + M)


def test_gemm_q4k_stacked_gate_up_m257(cuda):
    """The stacked gate|up weight (28672 x 4096) at M = 257: 256-token tiles with a one-token tail."""
    _check_gemm(cuda, qvx.Q4_K, 257, 28672, 4096, ALL16, seed=7300)


def test_gemm_q4k_ragged_256_token_tiles(cuda):
    """256-token tiles (the 4-wave kernel) with a ragged last row tile and a ragged last token tile:
    M = 1800, 14000 rows (55 columns of 256, the last of 176 rows)."""
    _check_gemm(cuda, qvx.Q4_K, 1800, 14000, 4096, ALL16, seed=7350)


def test_gemm_q4k_ffn_down_shape(cuda):
    """K = 14336 (a Q4_K ffn_down, 14336 -> 4096) at M = 2048 and M = 300."""
    _check_gemm(cuda, qvx.Q4_K, 2048, 4096, 14336, ALL16, seed=7400)
    _check_gemm(cuda, qvx.Q4_K, 300, 4096, 14336, ALL16, seed=7410)


def test_gemm_q6k_config_shapes(cuda):
    """Q6_K prefill weights of a Q4_K_M model: ffn_down 14336 -> 4096 and attn_v 4096 -> 1024."""
    _check_gemm(cuda, qvx.Q6_K, 2048, 4096, 14336, ALL16, seed=7500)
    _check_gemm(cuda, qvx.Q6_K, 512, 1024, 4096, ALL16, seed=7510, stride=13)


def _check_gemv_slice(cuda, t, rows, cols, m, seed, stride):
    W = qvx.empty_weight(t, rows, cols)
    qvx.fill_synthetic_t(W, t, rows, cols, seed=seed, scale_mul=1e-3)
    X = cuda.empty((m, cols), dtype=cuda.float32, device="cuda")
    qvx.fill_normal_t(X, seed=seed + 1)
    out = qvx.qmatmul_t(W, t, X, rows, cols)
    cuda.cuda.synchronize()
    idx = np.union1d(np.arange(0, rows, stride), [rows - 1])
    Wd = _row_slice(W.cpu().numpy(), t, rows, cols, idx).astype(np.float64)
    ref = X.cpu().numpy().astype(np.float64) @ Wd.T
    got = out.cpu().numpy()[:, idx]
    assert max_rel(got, ref) <= GEMV_TOL, (t, rows, cols, m)
    return W, X, out


def test_gemv_q6k_lm_head_m16(cuda):
    """Config 3's Q6_K LM head (4096 -> 128256) at M = 16, and each vector bit-identical to a
    one-vector call (qmatmul.hpp:31-32)."""
    t, rows, cols = qvx.Q6_K, 128256, 4096
    W, X, out = _check_gemv_slice(cuda, t, rows, cols, 16, seed=8100, stride=97)
    for v in (0, 5, 15):
        single = qvx.qmatmul_t(W, t, X[v], rows, cols)
        cuda.cuda.synchronize()
        np.testing.assert_array_equal(single.cpu().numpy().view(np.uint32), out[v].cpu().numpy().view(np.uint32))


@pytest.mark.parametrize("rows,cols,m", [(65573, 2048, 9), (70000, 6144, 16), (128256, 4096, 5), (128256, 4096, 2),
                                          (70000, 6144, 4)])
def test_gemv_q6k_tall_weights(cuda, rows, cols, m):
    """The batched Q6_K form on weights of 65536 rows or more (a workgroup streams ~30 tiles through
    its ring): ragged last tiles, a row of one 64-slot block and of several, 16-, 9-, 5-, 4- and
    2-vector launches; every vector bit-identical to a one-vector call."""
    t = qvx.Q6_K
    W, X, out = _check_gemv_slice(cuda, t, rows, cols, m, seed=8150 + m, stride=101)
    for v in range(m):
        single = qvx.qmatmul_t(W, t, X[v], rows, cols)
        cuda.cuda.synchronize()
        np.testing.assert_array_equal(single.cpu().numpy().view(np.uint32), out[v].cpu().numpy().view(np.uint32))


@pytest.mark.parametrize("rows,cols", [(14336, 4096), (4096, 14336)])
def test_gemv_q4k_m512(cuda, rows, cols):
    """qmatmul_n over 512 vectors at config 3's Q4_K shapes (64 launches of 8 vectors)."""
    _check_gemv_slice(cuda, qvx.Q4_K, rows, cols, 512, seed=8200 + rows, stride=37)


@pytest.mark.parametrize("t,rows,cols", [(qvx.Q8_0, 4096, 4096), (qvx.Q4_0, 11008, 4096), (qvx.Q4_0, 4096, 11008),
                                          (qvx.Q6_K, 4096, 14336), (qvx.Q6_K, 1024, 4096)])
@pytest.mark.parametrize("m", [8, 16])
def test_gemv_batched_config_shapes(cuda, t, rows, cols, m):
    """Batched GEMVs of the non-Q4_K formats at config 1 / 2 / 5 shapes (M = 8 and 16)."""
    _check_gemv_slice(cuda, t, rows, cols, m, seed=8300 + t + m, stride=7)
