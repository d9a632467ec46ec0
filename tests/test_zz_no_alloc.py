"""qvx_qgemm_f16_noalloc: the prefill GEMM with its temporaries in the library's fixed per-device
scratch array instead of an allocation.  Called through the C ABI and checked against
qvx_qgemm_f16 (the same kernels with a pool-allocated temporary) and against the fp64 oracle on a row
slice, on two calls in a row whose second input is smaller (the scratch keeps the first call's
contents), for every variant.  Both must match qvx_qgemm_f16 bit for bit: a K-split shape sums its
partial tiles in split order, so its result does not depend on the run.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
import qorvix_amd as qvx
from conftest import max_rel

pytestmark = pytest.mark.gpu

GEMM_TOL = 2e-2
I8_TOL = 1e-4


def _call(fn, cuda, W, t, X, rows, cols, variant):
    M = X.shape[0]
    out = cuda.full((M, rows), float("nan"), dtype=cuda.float32, device="cuda")
    rc = fn(out.data_ptr(), W.data_ptr(), t, X.data_ptr(), M, rows, cols, variant,
            cuda.cuda.current_stream().cuda_stream)
    assert rc == qvx.OK, qvx.strerror(rc)
    cuda.cuda.synchronize()
    return out.cpu().numpy()


def _case(cuda, M, rows, cols, seed, t=qvx.Q4_K):
    W = qvx.empty_weight(t, rows, cols)
    qvx.fill_synthetic_t(W, t, rows, cols, seed=seed, scale_mul=1e-3)
    X = cuda.empty((M, cols), dtype=cuda.float16, device="cuda")
    qvx.fill_normal_t(X, seed=seed + 1, mul=0.5)
    cuda.cuda.synchronize()
    idx = np.union1d(np.arange(0, rows, 29), [rows - 1])
    rb = qvx.row_bytes(t, cols)
    Wd = oracle.dequantize(t, W.cpu().numpy().reshape(rows, rb)[idx].reshape(-1), len(idx) * cols)
    Wd = Wd.reshape(len(idx), cols).astype(np.float64)
    return t, W, X, idx, Wd


@pytest.mark.parametrize("variant", [qvx.GEMM_BF16, qvx.GEMM_I8, qvx.GEMM_F16])
def test_noalloc_matches_allocating_gemm_on_two_calls(cuda, variant):
    lib = qvx.lib()
    # first call: 256-token tiles, no K split; second: smaller, 128-token tiles with a K split
    for n, (M, rows, cols) in enumerate(((1536, 14336, 4096), (128, 2048, 4096))):
        t, W, X, idx, Wd = _case(cuda, M, rows, cols, seed=900 + 10 * n + variant)
        got = _call(lib.qvx_qgemm_f16_noalloc, cuda, W, t, X, rows, cols, variant)
        want = _call(lib.qvx_qgemm_f16, cuda, W, t, X, rows, cols, variant)
        assert np.isfinite(got).all()
        np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))
        X32 = X.cpu().numpy().astype(np.float32)
        if variant == qvx.GEMM_I8:
            q, s, _ = oracle.quantize_q8_act(X32)
            ref = (q.astype(np.float64) * np.repeat(s.astype(np.float64), 32, axis=1)) @ Wd.T
            assert max_rel(got[:, idx], ref) <= I8_TOL
        else:
            assert max_rel(got[:, idx], X32.astype(np.float64) @ Wd.T) <= GEMM_TOL


@pytest.mark.parametrize("variant", [qvx.GEMM_BF16, qvx.GEMM_F16])
def test_noalloc_q6k_matches_allocating_gemm_on_two_calls(cuda, variant):
    """Q6_K (the Q4_K kernels' pipeline) through the no-allocation entry point: a 256-tile call with
    no K split (the bf16 copy of X, 56 MiB, in the scratch), then a smaller one whose four K splits
    keep their partial tiles and counters in the scratch the first call left behind; both within the
    GEMM tolerance of the fp64 oracle on a row slice.  The second is bit for bit the allocating
    call's; the first is a call the allocating entry point runs through the 16-bit weight and the
    plain GEMM instead (M >= 1024 on a weight of >= 32 Mi elements), so there the two agree within
    the GEMM tolerance of each other."""
    lib = qvx.lib()
    for n, (M, rows, cols) in enumerate(((2048, 4096, 14336), (128, 2048, 4096))):
        t, W, X, idx, Wd = _case(cuda, M, rows, cols, seed=950 + 10 * n + variant, t=qvx.Q6_K)
        got = _call(lib.qvx_qgemm_f16_noalloc, cuda, W, t, X, rows, cols, variant)
        want = _call(lib.qvx_qgemm_f16, cuda, W, t, X, rows, cols, variant)
        assert np.isfinite(got).all()
        if M >= 1024 and rows * cols >= 32 << 20:
            assert max_rel(got, want.astype(np.float64)) <= GEMM_TOL
        else:
            np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))
        X32 = X.cpu().numpy().astype(np.float64)
        assert max_rel(got[:, idx], X32 @ Wd.T) <= GEMM_TOL


@pytest.mark.parametrize("variant", [qvx.GEMM_BF16, qvx.GEMM_F16])
def test_noalloc_q6k_odd_blocks_matches_allocating_gemm(cuda, variant):
    """Q6_K rows of an odd number of super-blocks (cols 2304) run on the dequantising MFMA kernel
    k_qgemm_deq; at M = 128 its grid is small, so K splits and the partial tiles and counters live in
    the scratch.  Two calls, the second smaller; bit for bit the allocating call's, and within the GEMM
    tolerance of the fp64 oracle on a row slice."""
    lib = qvx.lib()
    for n, (M, rows, cols) in enumerate(((128, 4096, 2304), (64, 1024, 2304))):
        t, W, X, idx, Wd = _case(cuda, M, rows, cols, seed=990 + 10 * n + variant, t=qvx.Q6_K)
        got = _call(lib.qvx_qgemm_f16_noalloc, cuda, W, t, X, rows, cols, variant)
        want = _call(lib.qvx_qgemm_f16, cuda, W, t, X, rows, cols, variant)
        assert np.isfinite(got).all()
        np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))
        X32 = X.cpu().numpy().astype(np.float64)
        assert max_rel(got[:, idx], X32 @ Wd.T) <= GEMM_TOL


@pytest.mark.parametrize("t", [qvx.Q8_0, qvx.Q4_0])
@pytest.mark.parametrize("variant", [qvx.GEMM_BF16, qvx.GEMM_F16])
def test_noalloc_dequant16_types_match_allocating_gemm_on_two_calls(cuda, t, variant):
    """Q8_0 / Q4_0 (weight dequantised to 16 bits, then the plain MFMA GEMM) through the
    no-allocation entry point: first 2048 x 11008 x 4096, whose 90 MB 16-bit weight does not fit the
    scratch and runs in two panels of rows (128-token tiles, no K split, where the allocating call
    runs the whole weight on 256-token tiles: both add each output's K16 products in the same order,
    so the bits agree); then a smaller call with eight K splits, whose partial tiles and counters
    reuse the scratch the first call left behind.  Both bit for bit the allocating call's and within
    the GEMM tolerance of the fp64 oracle on a row slice."""
    lib = qvx.lib()
    for n, (M, rows, cols) in enumerate(((2048, 11008, 4096), (128, 2048, 4096))):
        t_, W, X, idx, Wd = _case(cuda, M, rows, cols, seed=970 + 10 * n + variant + t, t=t)
        got = _call(lib.qvx_qgemm_f16_noalloc, cuda, W, t, X, rows, cols, variant)
        want = _call(lib.qvx_qgemm_f16, cuda, W, t, X, rows, cols, variant)
        assert np.isfinite(got).all()
        np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))
        X32 = X.cpu().numpy().astype(np.float64)
        assert max_rel(got[:, idx], X32 @ Wd.T) <= GEMM_TOL


def test_noalloc_rejects_calls_past_its_scratch(cuda):
    """The bf16 copy of X needs 2 * M * cols bytes: past QVX_NOALLOC_SCRATCH_BYTES (64 MiB) the call is
    refused before any work, and the output is untouched; the fp16 variant needs no scratch."""
    lib = qvx.lib()
    t, rows, cols, M = qvx.Q4_K, 256, 4096, 8200  # 2 * 8200 * 4096 > 64 MiB
    W = qvx.empty_weight(t, rows, cols)
    qvx.fill_synthetic_t(W, t, rows, cols, seed=5, scale_mul=1e-3)
    X = cuda.zeros((M, cols), dtype=cuda.float16, device="cuda")
    out = cuda.full((M, rows), 3.0, dtype=cuda.float32, device="cuda")
    s = cuda.cuda.current_stream().cuda_stream
    assert lib.qvx_qgemm_f16_noalloc(out.data_ptr(), W.data_ptr(), t, X.data_ptr(), M, rows, cols,
                                     qvx.GEMM_BF16, s) == qvx.E_RANGE
    cuda.cuda.synchronize()
    assert bool((out == 3.0).all())
    assert lib.qvx_qgemm_f16_noalloc(out.data_ptr(), W.data_ptr(), t, X.data_ptr(), M, rows, cols,
                                     qvx.GEMM_F16, s) == qvx.OK
    cuda.cuda.synchronize()
    assert bool((out == 0.0).all())  # X is zero
