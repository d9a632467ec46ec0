"""qvx_qmatmul_n at encoder / prefill batch sizes (the many-vector Q4_K form, k_gemv_q4k_many) and the
bias epilogue (qvx_qmatmul_n_bias, the reference's wmatmulNBias).

The reference promises that qmatmulN is bit-identical to qmatmul per vector
(runtime/include/qorvix/runtime/qmatmul.hpp:31-32).  The many-vector form converts the activations
once and streams the weights once per 64 vectors; these tests hold every output to the one-vector
call's bits (qvx_qmatmul), and to the chunked batched forms' (a plan replay, which never takes the
many-vector form), at shapes whose one-vector geometry walks K in 4 and 16 ranges (including the
backward walks of even ranges), with ragged rows and a vector count that is not a multiple of 64.
The bias add is one fp32 add after the product: out == product + bias bit for bit.
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


@pytest.mark.parametrize("rows,cols,nvec", [(14336, 4096, 64), (4096, 14336, 100), (1000, 4096, 37),
                                            (1024, 2048, 16), (300, 768, 130)])
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
    # the chunked batched forms (a plan replay never takes the many-vector form) agree everywhere
    plan = decode.Plan()
    ref = cuda.full((nvec, rows), float("nan"), dtype=cuda.float32, device="cuda")
    plan.add(ref, decode.DevWeight(W, t, rows, cols), X, nvec)
    plan.instantiate()
    plan.launch(cuda.cuda.current_stream().cuda_stream)
    cuda.cuda.synchronize()
    assert cuda.equal(got.view(cuda.int32), ref.view(cuda.int32))


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
                                              (qvx.Q6_K, 512, 4096, 20), (qvx.F16, 300, 512, 5)])
def test_bias_is_one_add_after_the_product(cuda, t, rows, cols, nvec):
    """qvx_qmatmul_n_bias == qvx_qmatmul_n + bias, bit for bit, on the many-vector form (its epilogue)
    and on the routes that add the bias in a launch of its own; a null bias is qvx_qmatmul_n."""
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
