"""GPU parity of the decoder ops around the operator and of the fused calls (through the C ABI):

* qvx_rmsnorm / qvx_swiglu against the oracle's restatement of ops::rmsnorm / ops::swiglu
  (runtime/src/ops.cpp:8-13, 96-100; pinned bit-exact to the reference build in test_oracle.py);
* qvx_qmatmul_n_rmsnorm = W . rmsnorm(x): the norm folded into the GEMV kernels' activation
  conversion (Q4_K matrix-core forms, the integer-dot formats) and the standalone-norm route of the
  other types, against the fp64 product of exact dequantised weights and the oracle's normed x, at
  the GEMV bar (1e-3 max-relative); batches bit-identical to single vectors on the fused kernels;
* qvx_qmatmul_swiglu = silu(W_gate . xn) * (W_up . xn) over an interleaved gate|up weight, fused in
  the Q4_K epilogue and by product + standalone SwiGLU otherwise, against the oracle's SwiGLU of
  the fp64 products.  The bar: |y - ref| <= 1e-3 * (max|silu'| max|g| max|u| + max|silu(g)| max|u|),
  the first-order error of silu(g) u when g and u each carry the GEMV bar's error;
* qvx_interleave_rows16 byte for byte, and fused calls recorded in a plan and replayed as a graph.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
import qorvix_amd as qvx
from conftest import max_rel

pytestmark = pytest.mark.gpu

GEMV_TOL = 1e-3
EPS = 1e-5
SYNTH = {qvx.Q8_0: 0.01, qvx.Q4_0: 0.02, qvx.Q4_K: 1e-3, qvx.Q5_K: 1e-3, qvx.Q6_K: 1e-3}


def _weight(cuda, t, rows, cols, seed):
    if t in SYNTH:
        W = qvx.empty_weight(t, rows, cols)
        qvx.fill_synthetic_t(W, t, rows, cols, seed=seed, scale_mul=SYNTH[t])
        return W
    from test_gpu_kernels import random_weight
    w = random_weight(t, rows, cols, np.random.default_rng(seed))
    return cuda.from_numpy(w).cuda()


def _x(cuda, nvec, cols, seed, mul=1.0):
    X = cuda.empty((nvec, cols), dtype=cuda.float32, device="cuda")
    qvx.fill_normal_t(X, seed=seed, mul=mul)
    return X


def _normw(cuda, cols, seed):
    rng = np.random.default_rng(seed)
    return cuda.from_numpy((1.0 + 0.3 * rng.standard_normal(cols)).astype(np.float32)).cuda()


def _exact(W, t, Xn, rows, cols):
    return oracle.matmul_f64(W.cpu().numpy(), t, Xn.astype(np.float32), Xn.shape[0], rows, cols)


# ---- standalone ops ---------------------------------------------------------------------------------

@pytest.mark.parametrize("nvec,n", [(1, 4096), (3, 5120), (2, 7), (1, 14336)])
def test_rmsnorm_matches_oracle(cuda, nvec, n):
    x = _x(cuda, nvec, n, seed=n, mul=3.0)
    w = _normw(cuda, n, n + 1)
    y = qvx.rmsnorm_t(x, w, EPS)
    cuda.cuda.synchronize()
    ref = oracle.rmsnorm(x.cpu().numpy(), w.cpu().numpy(), EPS)
    # the sum of squares in double in another order: the scale may differ by an ulp
    np.testing.assert_allclose(y.cpu().numpy(), ref, rtol=5e-7, atol=0)


def test_swiglu_matches_oracle(cuda):
    rng = np.random.default_rng(3)
    g = (rng.standard_normal(100003) * 5).astype(np.float32)
    u = rng.standard_normal(g.size).astype(np.float32)
    y = qvx.swiglu_t(cuda.from_numpy(g).cuda(), cuda.from_numpy(u).cuda())
    cuda.cuda.synchronize()
    np.testing.assert_allclose(y.cpu().numpy(), oracle.swiglu(g, u), rtol=2e-6, atol=1e-30)


def test_interleave_rows16_layout(cuda):
    t, rows, cols = qvx.Q4_K, 48, 512
    a = _weight(cuda, t, rows, cols, 1)
    b = _weight(cuda, t, rows, cols, 2)
    il = qvx.interleave_rows16_t(a, b, t, rows, cols)
    cuda.cuda.synchronize()
    rb = qvx.row_bytes(t, cols)
    A, B, I = (z.cpu().numpy().reshape(-1, rb) for z in (a, b, il))
    for k in range(rows // 16):
        np.testing.assert_array_equal(I[32 * k:32 * k + 16], A[16 * k:16 * k + 16])
        np.testing.assert_array_equal(I[32 * k + 16:32 * k + 32], B[16 * k:16 * k + 16])
    with pytest.raises(qvx.QvxError):
        qvx.interleave_rows16_t(a, b, t, 40, cols)


# ---- GEMV with the norm folded in ---------------------------------------------------------------

# (type, rows, cols): fused on the Q4_K matrix-core forms and the integer-dot formats (cols % 512 ==
# 0), the standalone-norm route for Q4_K rows of 256 columns, F16 and Q4_1.
NORM_CASES = [(qvx.Q4_K, 1024, 4096), (qvx.Q4_K, 300, 4096), (qvx.Q4_K, 777, 2048), (qvx.Q6_K, 1024, 4096),
              (qvx.Q6_K, 515, 14336), (qvx.Q8_0, 600, 4096), (qvx.Q4_0, 256, 1024), (qvx.Q5_K, 333, 4096),
              (qvx.Q4_K, 64, 256), (qvx.F16, 300, 4096), (qvx.Q4_1, 200, 1024)]


@pytest.mark.parametrize("t,rows,cols", NORM_CASES)
@pytest.mark.parametrize("nvec", [1, 5])
def test_qmatmul_rmsnorm_parity(cuda, t, rows, cols, nvec):
    W = _weight(cuda, t, rows, cols, seed=rows + cols)
    X = _x(cuda, nvec, cols, seed=17, mul=2.0)
    nw = _normw(cuda, cols, 19)
    y = qvx.qmatmul_rmsnorm_t(W, t, X, nw, EPS, rows, cols)
    cuda.cuda.synchronize()
    xn = oracle.rmsnorm(X.cpu().numpy(), nw.cpu().numpy(), EPS)
    assert max_rel(y.cpu().numpy(), _exact(W, t, xn, rows, cols)) <= GEMV_TOL


@pytest.mark.parametrize("t,rows,cols", [(qvx.Q4_K, 1024, 4096), (qvx.Q6_K, 700, 4096), (qvx.Q8_0, 300, 2048),
                                         (qvx.Q4_K, 512, 8192)])
def test_qmatmul_rmsnorm_batches_bit_identical(cuda, t, rows, cols):
    """Every vector of a fused batch (2..8: the one-vector and batched matrix-core forms, the integer
    kernel's 2- and 4-vector launches) equals the single-vector fused call bit for bit."""
    W = _weight(cuda, t, rows, cols, seed=5)
    X = _x(cuda, 8, cols, seed=6)
    nw = _normw(cuda, cols, 7)
    single = np.stack([qvx.qmatmul_rmsnorm_t(W, t, X[v], nw, EPS, rows, cols).cpu().numpy() for v in range(8)])
    for n in (2, 3, 4, 8):
        got = qvx.qmatmul_rmsnorm_t(W, t, X[:n].contiguous(), nw, EPS, rows, cols).cpu().numpy()
        np.testing.assert_array_equal(got.view(np.uint32), single[:n].view(np.uint32))


@pytest.mark.parametrize("rows,cols", [(1024, 4096), (8200, 2048), (70000, 2048)])
def test_q6k_norm_batches_on_the_batched_form(cuda, rows, cols):
    """Q6_K batches with the RMSNorm prologue that the batched matrix-core form takes (the standalone
    norm into a temporary, then k_gemv_q6s: from 6 vectors on small weights, from 3 or 4 on weights of
    >= 8192 rows or columns, pairs on >= 65536 rows) equal the one-vector fused call (the VALU kernel
    folding the norm in) bit for bit, eagerly and replayed from a plan, whose workspace then holds
    the normalised activations and the block sums."""
    import ctypes as C
    t = qvx.Q6_K
    W = _weight(cuda, t, rows, cols, seed=rows + 3)
    X = _x(cuda, 8, cols, seed=8, mul=2.0)
    nw = _normw(cuda, cols, 9)
    single = np.stack([qvx.qmatmul_rmsnorm_t(W, t, X[v], nw, EPS, rows, cols).cpu().numpy() for v in range(8)])
    for n in (2, 3, 4, 6, 8):
        got = qvx.qmatmul_rmsnorm_t(W, t, X[:n].contiguous(), nw, EPS, rows, cols).cpu().numpy()
        np.testing.assert_array_equal(got.view(np.uint32), single[:n].view(np.uint32), err_msg=f"n={n}")
    lib = qvx.lib()
    out = cuda.full((8, rows), float("nan"), dtype=cuda.float32, device="cuda")
    plan = C.c_void_p()
    assert lib.qvx_plan_create(C.byref(plan)) == qvx.OK
    try:
        assert lib.qvx_plan_add_qmatmul_n_rmsnorm(plan, out.data_ptr(), W.data_ptr(), t, X.data_ptr(), nw.data_ptr(),
                                                  EPS, 8, rows, cols) == qvx.OK
        assert lib.qvx_plan_instantiate(plan) == qvx.OK
        s = cuda.cuda.current_stream().cuda_stream
        for rep in range(3):
            out.fill_(float("nan"))
            assert lib.qvx_plan_launch(plan, s) == qvx.OK
            cuda.cuda.synchronize()
            np.testing.assert_array_equal(out.cpu().numpy().view(np.uint32), single.view(np.uint32), err_msg=f"rep {rep}")
    finally:
        lib.qvx_plan_destroy(plan)
    xn = oracle.rmsnorm(X[:2].cpu().numpy(), nw.cpu().numpy(), EPS)
    idx = np.union1d(np.arange(0, rows, 97), [rows - 1])
    rb = qvx.row_bytes(t, cols)
    wsl = W.cpu().numpy().reshape(rows, rb)[idx].reshape(-1)
    ref = oracle.matmul_f64(wsl, t, xn.astype(np.float32), 2, len(idx), cols)
    assert max_rel(single[:2][:, idx], ref) <= GEMV_TOL


def test_qmatmul_rmsnorm_checks(cuda):
    W = _weight(cuda, qvx.Q4_K, 64, 512, 1)
    X = _x(cuda, 1, 512, 2)
    out = cuda.empty(64, device="cuda")
    s = cuda.cuda.current_stream().cuda_stream
    assert qvx.qmatmul_n_rmsnorm(out.data_ptr(), W.data_ptr(), qvx.Q4_K, X.data_ptr(), None, EPS, 1, 64, 512, s) == qvx.E_NULL
    assert qvx.qmatmul_n_rmsnorm(out.data_ptr(), W.data_ptr(), 99, X.data_ptr(), X.data_ptr(), EPS, 1, 64, 512, s) == qvx.E_TYPE
    assert qvx.qmatmul_n_rmsnorm(out.data_ptr(), W.data_ptr(), qvx.Q4_K, X.data_ptr(), X.data_ptr(), EPS, 0, 64, 512, s) == qvx.E_NVEC


# ---- GEMV with the SwiGLU epilogue ------------------------------------------------------------------

def _swiglu_ref(cuda, t, Wg, Wu, X, nw, ffn, cols):
    x = X.cpu().numpy()
    xn = oracle.rmsnorm(x, nw.cpu().numpy(), EPS) if nw is not None else x
    g = _exact(Wg, t, xn, ffn, cols)
    u = _exact(Wu, t, xn, ffn, cols)
    ref = oracle.swiglu(g.astype(np.float32), u.astype(np.float32)).astype(np.float64)
    z = np.linspace(-12, 12, 4001)
    dsilu = np.abs(1 / (1 + np.exp(-z)) * (1 + z * (1 - 1 / (1 + np.exp(-z))))).max()
    silu_g = np.abs(g / (1 + np.exp(-g))).max()
    bound = GEMV_TOL * (dsilu * np.abs(g).max() * np.abs(u).max() + silu_g * np.abs(u).max())
    return ref, bound


@pytest.mark.parametrize("t,ffn,cols", [(qvx.Q4_K, 14336, 4096), (qvx.Q4_K, 1040, 2048), (qvx.Q4_K, 48, 512),
                                        (qvx.Q6_K, 1024, 4096), (qvx.Q4_K, 256, 256)])
@pytest.mark.parametrize("nvec", [1, 3, 8])
@pytest.mark.parametrize("norm", [True, False])
def test_qmatmul_swiglu_parity(cuda, t, ffn, cols, nvec, norm):
    Wg = _weight(cuda, t, ffn, cols, seed=11)
    Wu = _weight(cuda, t, ffn, cols, seed=12)
    Wgu = qvx.interleave_rows16_t(Wg, Wu, t, ffn, cols)
    X = _x(cuda, nvec, cols, seed=13, mul=1.5)
    nw = _normw(cuda, cols, 14) if norm else None
    y = qvx.qmatmul_swiglu_t(Wgu, t, X, ffn, cols, norm_w=nw, eps=EPS)
    cuda.cuda.synchronize()
    ref, bound = _swiglu_ref(cuda, t, Wg, Wu, X, nw, ffn, cols)
    err = float(np.abs(y.cpu().numpy() - ref).max())
    assert err <= bound, (err, bound)


def test_qmatmul_swiglu_batches_bit_identical(cuda):
    t, ffn, cols = qvx.Q4_K, 14336, 4096
    Wgu = qvx.interleave_rows16_t(_weight(cuda, t, ffn, cols, 21), _weight(cuda, t, ffn, cols, 22), t, ffn, cols)
    X = _x(cuda, 8, cols, seed=23)
    nw = _normw(cuda, cols, 24)
    single = np.stack([qvx.qmatmul_swiglu_t(Wgu, t, X[v], ffn, cols, nw, EPS).cpu().numpy() for v in range(8)])
    for n in (2, 3, 5, 8):
        got = qvx.qmatmul_swiglu_t(Wgu, t, X[:n].contiguous(), ffn, cols, nw, EPS).cpu().numpy()
        np.testing.assert_array_equal(got.view(np.uint32), single[:n].view(np.uint32))


def test_qmatmul_swiglu_checks(cuda):
    W = _weight(cuda, qvx.Q4_K, 64, 512, 1)
    X = _x(cuda, 1, 512, 2)
    out = cuda.empty(32, device="cuda")
    s = cuda.cuda.current_stream().cuda_stream
    assert qvx.qmatmul_swiglu(out.data_ptr(), W.data_ptr(), qvx.Q4_K, X.data_ptr(), None, EPS, 1, 24, 512, s) == qvx.E_SHAPE
    assert qvx.qmatmul_swiglu(out.data_ptr(), W.data_ptr(), qvx.Q4_K, X.data_ptr(), None, EPS, 0, 32, 512, s) == qvx.E_NVEC


# ---- fused calls in a plan ----------------------------------------------------------------------------

def test_plan_with_fused_calls_replays_like_eager(cuda):
    """A plan of a layer's fused calls (q|k with the attention norm, v (Q6_K) with it, gate|up with the
    FFN norm and SwiGLU, down on the SwiGLU output) replays as a graph with the eager results, three
    times in a row; a fused call no kernel folds in is refused at record time."""
    import ctypes as C
    lib = qvx.lib()
    d, ffn = 4096, 14336
    Wqk = _weight(cuda, qvx.Q4_K, 5120, d, 31)
    Wv = _weight(cuda, qvx.Q6_K, 1024, d, 32)
    Wgu = qvx.interleave_rows16_t(_weight(cuda, qvx.Q4_K, ffn, d, 33), _weight(cuda, qvx.Q4_K, ffn, d, 34),
                                  qvx.Q4_K, ffn, d)
    Wd = _weight(cuda, qvx.Q6_K, d, ffn, 35)
    x = _x(cuda, 1, d, 36)
    n1, n2 = _normw(cuda, d, 37), _normw(cuda, d, 38)
    qk = cuda.empty(5120, device="cuda")
    v = cuda.empty(1024, device="cuda")
    h = cuda.empty(ffn, device="cuda")
    o = cuda.empty(d, device="cuda")
    plan = C.c_void_p()
    assert lib.qvx_plan_create(C.byref(plan)) == qvx.OK
    try:
        assert lib.qvx_plan_add_qmatmul_n_rmsnorm(plan, qk.data_ptr(), Wqk.data_ptr(), qvx.Q4_K, x.data_ptr(),
                                                  n1.data_ptr(), EPS, 1, 5120, d) == qvx.OK
        assert lib.qvx_plan_add_qmatmul_n_rmsnorm(plan, v.data_ptr(), Wv.data_ptr(), qvx.Q6_K, x.data_ptr(),
                                                  n1.data_ptr(), EPS, 1, 1024, d) == qvx.OK
        assert lib.qvx_plan_add_qmatmul_swiglu(plan, h.data_ptr(), Wgu.data_ptr(), qvx.Q4_K, x.data_ptr(),
                                               n2.data_ptr(), EPS, 1, ffn, d) == qvx.OK
        assert lib.qvx_plan_add_qmatmul_n(plan, o.data_ptr(), Wd.data_ptr(), qvx.Q6_K, h.data_ptr(), 1, d, ffn) == qvx.OK
        Wf16 = _weight(cuda, qvx.F16, 64, d, 39)
        tmp = cuda.empty(64, device="cuda")
        assert lib.qvx_plan_add_qmatmul_n_rmsnorm(plan, tmp.data_ptr(), Wf16.data_ptr(), qvx.F16, x.data_ptr(),
                                                  n1.data_ptr(), EPS, 1, 64, d) == qvx.E_SHAPE
        s = cuda.cuda.current_stream().cuda_stream
        assert lib.qvx_plan_run_eager(plan, s) == qvx.OK
        cuda.cuda.synchronize()
        eager = [z.cpu().numpy().copy() for z in (qk, v, h, o)]
        assert lib.qvx_plan_instantiate(plan) == qvx.OK
        for _ in range(3):
            for z in (qk, v, h, o):
                z.fill_(float("nan"))
            cuda.cuda.synchronize()
            assert lib.qvx_plan_launch(plan, s) == qvx.OK
            cuda.cuda.synchronize()
            for z, e in zip((qk, v, h, o), eager):
                np.testing.assert_array_equal(z.cpu().numpy().view(np.uint32), e.view(np.uint32))
    finally:
        lib.qvx_plan_destroy(plan)
    # and the eager layer against the oracle
    xn1 = oracle.rmsnorm(x.cpu().numpy(), n1.cpu().numpy(), EPS)
    assert max_rel(eager[0], _exact(Wqk, qvx.Q4_K, xn1, 5120, d)[0]) <= GEMV_TOL
    assert max_rel(eager[1], _exact(Wv, qvx.Q6_K, xn1, 1024, d)[0]) <= GEMV_TOL
    assert max_rel(eager[3], _exact(Wd, qvx.Q6_K, eager[2][None, :], d, ffn)[0]) <= GEMV_TOL
