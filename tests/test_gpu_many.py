"""qvx_qmatmul_n at encoder / prefill batch sizes (the many-vector Q4_K form, k_gemv_q4k_many) and the
bias epilogue (qvx_qmatmul_n_bias, the reference's wmatmulNBias).

The reference promises that qmatmulN is bit-identical to qmatmul per vector
(runtime/include/qorvix/runtime/qmatmul.hpp:31-32).  The many-vector form converts the activations
once and streams the weights once per 64 vectors (once per 16, with the K ranges split over
workgroups, up to 32 vectors; it takes batches from 12 vectors on weights of >= 32 Mi elements and
from 24 on smaller ones); these tests hold every output to the one-vector call's bits
(qvx_qmatmul), and to the chunked batched forms' (calls of 8 vectors), at shapes whose one-vector
geometry walks K in 1, 4 and 16 ranges (including the backward walks of even ranges), with ragged
rows and vector counts on both sides of 32 and not multiples of 16 or 64.  A plan replays the
many-vector form from its own workspace, also for calls in one fork.  The bias add is one fp32 add
after the product: out == product + bias bit for bit.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
import qorvix_amd as qvx
from conftest import max_rel
from qorvix_amd import decode

pytestmark = pytest.mark.gpu


def _weight(cuda, t, rows, cols, seed):
    W = qvx.empty_weight(t, rows, cols)
    qvx.fill_synthetic_t(W, t, rows, cols, seed=seed, scale_mul=1e-3)
    return W


def _many(cuda, W, t, X, rows, cols, bias=None):
    n = X.shape[0]
    out = cuda.full((n, rows), float("nan"), dtype=cuda.float32, device="cuda")
    s = cuda.cuda.current_stream().cuda_stream
    if bias is None:
        rc = qvx.qmatmul_n(out.data_ptr(), W.data_ptr(), t, X.data_ptr(), n, rows, cols, s)
    else:
        rc = qvx.qmatmul_n_bias(out.data_ptr(), W.data_ptr(), t, X.data_ptr(), bias.data_ptr(), n, rows, cols, s)
    assert rc == qvx.OK, qvx.strerror(rc)
    return out


def _chunked(cuda, W, t, X, rows, cols):
    """qvx_qmatmul_n in calls of 8 vectors: the chunked batched forms."""
    n = X.shape[0]
    ref = cuda.full((n, rows), float("nan"), dtype=cuda.float32, device="cuda")
    s = cuda.cuda.current_stream().cuda_stream
    for v0 in range(0, n, 8):
        k = min(8, n - v0)
        rc = qvx.qmatmul_n(ref[v0].data_ptr(), W.data_ptr(), t, X[v0].data_ptr(), k, rows, cols, s)
        assert rc == qvx.OK, qvx.strerror(rc)
    return ref


@pytest.mark.parametrize("rows,cols,nvec", [(14336, 4096, 64), (4096, 14336, 100), (1000, 4096, 37),
                                            (1024, 2048, 24), (300, 768, 130), (4096, 14336, 16),
                                            (14336, 4096, 12), (14336, 4096, 29), (128256, 4096, 20),
                                            (4096, 4096, 32)])
def test_many_bit_identical_to_single_vector_calls(cuda, rows, cols, nvec):
    t = qvx.Q4_K
    W = _weight(cuda, t, rows, cols, seed=rows + nvec)
    X = qvx.fill_normal_t(cuda.empty((nvec, cols), dtype=cuda.float32, device="cuda"), seed=cols + nvec)
    got = _many(cuda, W, t, X, rows, cols)
    one = cuda.empty(rows, dtype=cuda.float32, device="cuda")
    for v in range(0, nvec, max(1, nvec // 9)):
        assert qvx.qmatmul(one.data_ptr(), W.data_ptr(), t, X[v].data_ptr(), rows, cols) == qvx.OK
        cuda.cuda.synchronize()
        assert cuda.equal(got[v].view(cuda.int32), one.view(cuda.int32)), v
    # the chunked batched forms agree everywhere
    ref = _chunked(cuda, W, t, X, rows, cols)
    cuda.cuda.synchronize()
    assert cuda.equal(got.view(cuda.int32), ref.view(cuda.int32))


def test_plan_replays_many_vector_calls(cuda):
    """A plan's many-vector calls (in order, and two in one fork, which need disjoint workspace
    slices) replay bit-identically to the direct calls, several times with eager work between."""
    t = qvx.Q4_K
    shapes = [(4096, 14336, 16), (14336, 4096, 48), (4096, 4096, 24)]
    Ws = [_weight(cuda, t, r, c, seed=40 + i) for i, (r, c, n) in enumerate(shapes)]
    Xs = [qvx.fill_normal_t(cuda.empty((n, c), dtype=cuda.float32, device="cuda"), seed=50 + i)
          for i, (r, c, n) in enumerate(shapes)]
    want = [_many(cuda, W, t, X, r, c) for W, X, (r, c, n) in zip(Ws, Xs, shapes)]
    outs = [cuda.full((n, r), float("nan"), dtype=cuda.float32, device="cuda") for (r, c, n) in shapes]
    plan = decode.Plan()
    plan.add(outs[0], decode.DevWeight(Ws[0], t, *shapes[0][:2]), Xs[0], shapes[0][2])
    plan.fork()
    for i in (1, 2):
        plan.add(outs[i], decode.DevWeight(Ws[i], t, *shapes[i][:2]), Xs[i], shapes[i][2])
    plan.join()
    plan.instantiate()
    s = cuda.cuda.current_stream().cuda_stream
    for rep in range(3):
        for o in outs:
            o.fill_(float("nan"))
        plan.launch(s)
        cuda.cuda.synchronize()
        for i in range(3):
            assert cuda.equal(outs[i].view(cuda.int32), want[i].view(cuda.int32)), (rep, i)
    plan.close()


def test_plan_replays_split_q4k_calls(cuda):
    """The split Q4_K form in a plan (range partials in the plan's workspace, with a bias on one call):
    replays bit-identical to the direct calls, several times."""
    t = qvx.Q4_K
    shapes = [(4096, 14336, 8), (1024, 4096, 16)]
    Ws = [_weight(cuda, t, r, c, seed=80 + i) for i, (r, c, n) in enumerate(shapes)]
    Xs = [qvx.fill_normal_t(cuda.empty((n, c), dtype=cuda.float32, device="cuda"), seed=90 + i)
          for i, (r, c, n) in enumerate(shapes)]
    want = [_many(cuda, W, t, X, r, c) for W, X, (r, c, n) in zip(Ws, Xs, shapes)]
    outs = [cuda.full((n, r), float("nan"), dtype=cuda.float32, device="cuda") for (r, c, n) in shapes]
    plan = decode.Plan()
    for i in range(2):
        plan.add(outs[i], decode.DevWeight(Ws[i], t, *shapes[i][:2]), Xs[i], shapes[i][2])
    plan.instantiate()
    s = cuda.cuda.current_stream().cuda_stream
    for rep in range(3):
        for o in outs:
            o.fill_(float("nan"))
        plan.launch(s)
        cuda.cuda.synchronize()
        for i in range(2):
            assert cuda.equal(outs[i].view(cuda.int32), want[i].view(cuda.int32)), (rep, i)
    plan.close()


def test_plan_replays_batched_q6k_calls(cuda):
    """The batched Q6_K form in a plan (block sums in the plan's workspace, rows of several blocks;
    a one-block call needs none): replays bit-identical to the direct calls, several times."""
    t = qvx.Q6_K
    shapes = [(4096, 14336, 8), (1000, 4096, 16), (4096, 2048, 6)]
    Ws = [_weight(cuda, t, r, c, seed=60 + i) for i, (r, c, n) in enumerate(shapes)]
    Xs = [qvx.fill_normal_t(cuda.empty((n, c), dtype=cuda.float32, device="cuda"), seed=70 + i)
          for i, (r, c, n) in enumerate(shapes)]
    want = [_many(cuda, W, t, X, r, c) for W, X, (r, c, n) in zip(Ws, Xs, shapes)]
    outs = [cuda.full((n, r), float("nan"), dtype=cuda.float32, device="cuda") for (r, c, n) in shapes]
    plan = decode.Plan()
    for i in range(3):
        plan.add(outs[i], decode.DevWeight(Ws[i], t, *shapes[i][:2]), Xs[i], shapes[i][2])
    plan.instantiate()
    s = cuda.cuda.current_stream().cuda_stream
    for rep in range(3):
        for o in outs:
            o.fill_(float("nan"))
        plan.launch(s)
        cuda.cuda.synchronize()
        for i in range(3):
            assert cuda.equal(outs[i].view(cuda.int32), want[i].view(cuda.int32)), (rep, i)
    plan.close()


def test_plan_adds_q6k_block_sums_in_the_kernel(cuda):
    """Batched Q6_K calls of <= 8 vectors whose workgroups take at most two 32-row tiles add their
    block sums in the kernel inside a plan (per-tile counters in the plan's workspace, zeroed at
    instantiation, left zero by the tile's last workgroup); the direct calls use the sum launch.
    Shapes: one and two tiles a workgroup, 2, 4 and 8 blocks a row, ragged rows, 3 to 8 vectors,
    two calls in one fork (disjoint counter slices); every replay bit-identical to the direct call."""
    t = qvx.Q6_K
    shapes = [(1024, 4096, 8), (8192, 4096, 7), (1000, 8192, 4), (2048, 8192, 5), (500, 16384, 3)]
    Ws = [_weight(cuda, t, r, c, seed=100 + i) for i, (r, c, n) in enumerate(shapes)]
    Xs = [qvx.fill_normal_t(cuda.empty((n, c), dtype=cuda.float32, device="cuda"), seed=110 + i)
          for i, (r, c, n) in enumerate(shapes)]
    want = [_many(cuda, W, t, X, r, c) for W, X, (r, c, n) in zip(Ws, Xs, shapes)]
    outs = [cuda.full((n, r), float("nan"), dtype=cuda.float32, device="cuda") for (r, c, n) in shapes]
    plan = decode.Plan()
    for i in range(3):
        plan.add(outs[i], decode.DevWeight(Ws[i], t, *shapes[i][:2]), Xs[i], shapes[i][2])
    plan.fork()
    for i in (3, 4):
        plan.add(outs[i], decode.DevWeight(Ws[i], t, *shapes[i][:2]), Xs[i], shapes[i][2])
    plan.join()
    plan.instantiate()
    s = cuda.cuda.current_stream().cuda_stream
    for rep in range(4):
        for o in outs:
            o.fill_(float("nan"))
        plan.launch(s)
        cuda.cuda.synchronize()
        for i in range(len(shapes)):
            assert cuda.equal(outs[i].view(cuda.int32), want[i].view(cuda.int32)), (rep, i)
    plan.close()


def test_many_matches_oracle_at_encoder_batch(cuda):
    """BASELINE's Q4_K 14336 x 4096 weight at 512 vectors (the verdict's encoder-size point) against the
    fp64 oracle on a row slice, within the GEMV bar."""
    t, rows, cols, nvec = qvx.Q4_K, 14336, 4096, 512
    W = _weight(cuda, t, rows, cols, seed=77)
    X = qvx.fill_normal_t(cuda.empty((nvec, cols), dtype=cuda.float32, device="cuda"), seed=78)
    got = _many(cuda, W, t, X, rows, cols).cpu().numpy()
    assert np.isfinite(got).all()
    rb = qvx.row_bytes(t, cols)
    idx = np.union1d(np.arange(0, rows, 131), [rows - 1])
    wsl = W.cpu().numpy().reshape(rows, rb)[idx].reshape(-1)
    ref = oracle.matmul_f64(wsl, t, X.cpu().numpy(), nvec, len(idx), cols)
    assert max_rel(got[:, idx], ref) <= 1e-3


@pytest.mark.parametrize("t,rows,cols,nvec", [(qvx.Q4_K, 1000, 4096, 40), (qvx.Q4_K, 512, 4096, 3),
                                              (qvx.Q4_K, 700, 14336, 8), (qvx.Q6_K, 512, 4096, 20),
                                              (qvx.F16, 300, 512, 5)])
def test_bias_is_one_add_after_the_product(cuda, t, rows, cols, nvec):
    """qvx_qmatmul_n_bias == qvx_qmatmul_n + bias, bit for bit, on the many-vector form (its epilogue),
    the split Q4_K form (its sum launch) and on the routes that add the bias in a launch of its own; a
    null bias is qvx_qmatmul_n."""
    if t == qvx.F16:
        W = cuda.randn(rows * cols, device="cuda").to(cuda.float16).view(cuda.uint8)
    else:
        W = _weight(cuda, t, rows, cols, seed=5 + t)
    X = qvx.fill_normal_t(cuda.empty((nvec, cols), dtype=cuda.float32, device="cuda"), seed=9)
    bias = qvx.fill_normal_t(cuda.empty(rows, dtype=cuda.float32, device="cuda"), seed=10)
    plain = _many(cuda, W, t, X, rows, cols)
    with_b = _many(cuda, W, t, X, rows, cols, bias)
    cuda.cuda.synchronize()
    assert cuda.equal(with_b.view(cuda.int32), (plain + bias[None, :]).view(cuda.int32))
    out = cuda.full((nvec, rows), float("nan"), dtype=cuda.float32, device="cuda")
    assert qvx.qmatmul_n_bias(out.data_ptr(), W.data_ptr(), t, X.data_ptr(), 0, nvec, rows, cols,
                              cuda.cuda.current_stream().cuda_stream) == qvx.OK
    cuda.cuda.synchronize()
    assert cuda.equal(out.view(cuda.int32), plain.view(cuda.int32))
