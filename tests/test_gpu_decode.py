"""GPU tests of the decode-step plan: a token's GEMVs captured into one HIP graph replay to the same
bits as the eager calls (several replays, with other work and synchronisations between them), and
their outputs agree with the oracle."""
from __future__ import annotations

import numpy as np
import pytest

import oracle
import qorvix_amd as qvx
from conftest import max_rel
from qorvix_amd import decode

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def small_model(cuda):
    # two Llama-3-8B layers + the LM head: every projection shape and type of the full sweep
    return decode.Model.synthetic(n_layers=2, lm_head=True, seed=7)


@pytest.mark.parametrize("m,concurrent", [(1, True), (8, True), (1, False)])
def test_plan_replays_match_eager(cuda, small_model, m, concurrent):
    torch = cuda
    step = decode.DecodeStep(small_model, m, seed=m, concurrent=concurrent)
    assert len(step.plan) == 2 * 7 + 1
    s = torch.cuda.current_stream().cuda_stream
    step.run_eager(s)
    torch.cuda.synchronize()
    ref = [y.clone() for _, _, y in step.outputs]
    for rep in range(3):
        for _, _, y in step.outputs:
            y.fill_(float("nan"))
        noise = torch.randn(1 << 20, device="cuda")  # eager work between replays
        float(noise.sum())
        step.replay(s)
        torch.cuda.synchronize()
        for (l, name, y), r in zip(step.outputs, ref):
            assert torch.equal(y.view(torch.int32), r.view(torch.int32)), (rep, l, name)
    step.plan.close()


@pytest.mark.parametrize("stacked", [False, True])
def test_grouped_plan_matches_plain(cuda, small_model, stacked):
    """q/k/v and gate/up as grouped calls, or q|k stacked and grouped with v (4 launches a layer either
    way): every output bit-identical to the ungrouped plan's on the same weights, on every replay."""
    torch = cuda
    model = small_model.fused() if stacked else small_model
    plain = decode.DecodeStep(model, 1, seed=4)
    grouped = decode.DecodeStep(model, 1, seed=4, grouped=True)
    assert len(grouped.plan) == 2 * 4 + 1
    s = torch.cuda.current_stream().cuda_stream
    plain.replay(s)
    torch.cuda.synchronize()
    for rep in range(3):
        for _, _, y in grouped.outputs:
            y.fill_(float("nan"))
        float(torch.randn(1 << 20, device="cuda").sum())
        grouped.replay(s)
        torch.cuda.synchronize()
        for (l, name, y), (_, _, r) in zip(grouped.outputs, plain.outputs):
            assert torch.equal(y.view(torch.int32), r.view(torch.int32)), (rep, l, name)
    plain.plan.close()
    grouped.plan.close()


def test_fused_grouped_step_matches_fused(cuda, small_model):
    """The fused decode step with q|k and v on the normed state as one grouped launch (4 launches a
    layer): every output bit-identical to the 5-launch step's."""
    torch = cuda
    fops = small_model.fused_ops()
    five = decode.FusedDecodeStep(fops, 1, seed=6)
    four = decode.FusedDecodeStep(fops, 1, seed=6, grouped=True)
    assert five.launches() == 2 * 5 + 1 and four.launches() == 2 * 4 + 1
    s = torch.cuda.current_stream().cuda_stream
    five.replay(s)
    torch.cuda.synchronize()
    ref = {k: v.clone() for k, v in five.out.items()}
    ref_h, ref_lg = five.h.clone(), five.logits.clone()
    for rep in range(3):
        for v in list(four.out.values()) + [four.h, four.logits]:
            v.fill_(float("nan"))
        float(torch.randn(1 << 20, device="cuda").sum())
        four.replay(s)
        torch.cuda.synchronize()
        for k, r in ref.items():
            assert torch.equal(four.out[k].view(torch.int32), r.view(torch.int32)), (rep, k)
        assert torch.equal(four.h.view(torch.int32), ref_h.view(torch.int32)), rep
        assert torch.equal(four.logits.view(torch.int32), ref_lg.view(torch.int32)), rep
    five.plan.close()
    four.plan.close()


def test_plan_outputs_match_oracle(cuda, small_model):
    torch = cuda
    step = decode.DecodeStep(small_model, 2, seed=3)
    step.replay(torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    X = {k: v.cpu().numpy() for k, v in step.inputs.items()}
    for (l, name, y), (_, _, rows, cols, t, src) in zip(step.outputs, decode.sweep_specs(2, True)):
        w = small_model.layers[l][name] if l < 2 else small_model.lm_head
        rb = qvx.row_bytes(t, cols)
        r0 = (rows // 3) & ~15
        nr = 48
        wrows = w.data[r0 * rb:(r0 + nr) * rb].cpu().numpy()
        ref = oracle.matmul_f64(wrows, t, X[src], 2, nr, cols)
        assert max_rel(y[:, r0:r0 + nr].cpu().numpy(), ref) <= 1e-3, (l, name)
    step.plan.close()


def test_plan_state_and_argument_errors(cuda):
    torch = cuda
    p = decode.Plan()
    W = qvx.empty_weight(qvx.Q4_K, 16, 256)
    x = torch.zeros(256, device="cuda")
    y = torch.zeros(16, device="cuda")
    with pytest.raises(qvx.QvxError) as e:
        p.launch(0)
    assert e.value.code == qvx.E_STATE
    lib = qvx.lib()
    assert lib.qvx_plan_join(p._h) == qvx.E_STATE
    assert lib.qvx_plan_fork(p._h) == qvx.OK
    assert lib.qvx_plan_fork(p._h) == qvx.E_STATE
    assert lib.qvx_plan_join(p._h) == qvx.OK
    assert lib.qvx_plan_add_qmatmul_n(p._h, y.data_ptr(), W.data_ptr(), 99, x.data_ptr(), 1, 16, 256) == qvx.E_TYPE
    assert lib.qvx_plan_add_qmatmul_n(p._h, y.data_ptr(), W.data_ptr(), qvx.Q4_K, x.data_ptr(), 1, 16, 200) == qvx.E_SHAPE
    assert lib.qvx_plan_add_qmatmul_n(p._h, y.data_ptr(), W.data_ptr(), qvx.Q4_K, x.data_ptr(), 0, 16, 256) == qvx.E_NVEC
    assert lib.qvx_plan_add_qmatmul_n(p._h, y.data_ptr(), W.data_ptr(), qvx.Q4_K, x.data_ptr(), 1, 0, 256) == qvx.OK
    assert len(p) == 0
    p.add(y, decode.DevWeight(W, qvx.Q4_K, 16, 256), x, 1)
    p.instantiate()
    assert lib.qvx_plan_add_qmatmul_n(p._h, y.data_ptr(), W.data_ptr(), qvx.Q4_K, x.data_ptr(), 1, 16, 256) == qvx.E_STATE
    assert lib.qvx_plan_fork(p._h) == qvx.E_STATE
    p.launch(torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    p.close()


@pytest.mark.parametrize("m", [16, 130])
def test_prefill_outputs_match_oracle(cuda, small_model, m):
    """The batched prefill: every projection of the last layer (the outputs are reused across layers)
    within the GEMM tolerance of the oracle on a slice of rows, the Q4_K ones on the raw-block MFMA
    kernel and the Q6_K ones on the dequantising MFMA kernel; the LM head on the last position within
    the GEMV tolerance."""
    torch = cuda
    step = decode.PrefillStep(small_model, m, seed=m)
    step.run(torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    X = {k: v.cpu().numpy().astype(np.float32) for k, v in step.inputs.items()}
    last = small_model.layers[-1]
    for name, rows, cols, t, src in decode.LAYER_SPECS:
        w = last[name]
        assert w.type == t
        rb = qvx.row_bytes(t, cols)
        r0 = (rows // 3) & ~15
        nr = 48
        wrows = w.data[r0 * rb:(r0 + nr) * rb].cpu().numpy()
        ref = oracle.matmul_f64(wrows, t, X[src], m, nr, cols)
        assert max_rel(step.outputs[name][:, r0:r0 + nr].cpu().numpy(), ref) <= 2e-2, name
    head = small_model.lm_head
    rb = qvx.row_bytes(head.type, head.cols)
    wrows = head.data[:64 * rb].cpu().numpy()
    ref = oracle.matmul_f64(wrows, head.type, step.last.cpu().numpy(), 1, 64, head.cols)
    assert max_rel(step.logits[:, :64].cpu().numpy(), ref) <= 1e-3
    assert step.flops() == 2 * m * sum(w.rows * w.cols for l in small_model.layers for w in l.values()) + \
        2 * head.rows * head.cols


@pytest.mark.parametrize("variant", [qvx.GEMM_F16, qvx.GEMM_BF16])
def test_prefill_graph_replays_match_eager(cuda, small_model, variant):
    """The whole prefill step (Q4_K and Q6_K GEMMs, the LM head GEMV) captured into one graph:
    every replay, with other work and synchronisations between them, is bit-identical to the eager
    run (split-K partial sums are added in split order, and the no-allocation entry point the graph
    records runs the allocating one's kernels)."""
    torch = cuda
    step = decode.PrefillStep(small_model, 130, seed=17, variant=variant)
    s = torch.cuda.current_stream().cuda_stream
    step.run(s)
    torch.cuda.synchronize()
    ref = {k: v.clone() for k, v in step.outputs.items()}
    ref_logits = step.logits.clone()
    step.capture()
    for rep in range(3):
        for v in step.outputs.values():
            v.fill_(float("nan"))
        step.logits.fill_(float("nan"))
        noise = torch.randn(1 << 20, device="cuda")  # eager work between replays
        float(noise.sum())
        step.replay()
        torch.cuda.synchronize()
        for k, v in step.outputs.items():
            assert torch.equal(v.view(torch.int32), ref[k].view(torch.int32)), (rep, k)
        assert torch.equal(step.logits.view(torch.int32), ref_logits.view(torch.int32)), rep


@pytest.mark.parametrize("m", [1, 8])
def test_fused_plan_matches_unfused(cuda, small_model, m):
    """The stacked q|k and gate|up weights: one GEMV each gives the parts' outputs within the GEMV
    tolerance of the separate calls (their launch geometry differs, so not bit for bit); v, o, down
    and the LM head run the same calls and match bit for bit."""
    torch = cuda
    fused = small_model.fused()
    a = decode.DecodeStep(small_model, m, seed=21)
    b = decode.DecodeStep(fused, m, seed=21)
    assert len(b.plan) == 2 * 5 + 1
    s = torch.cuda.current_stream().cuda_stream
    a.replay(s)
    b.replay(s)
    torch.cuda.synchronize()
    ya = {(l, n): y for l, n, y in a.outputs}
    for l, n, y in b.outputs:
        if n in fused.parts:
            r0 = 0
            for part, rows in fused.parts[n]:
                ref = ya[(l, part)].cpu().numpy()
                assert max_rel(y[:, r0:r0 + rows].cpu().numpy(), ref) <= 1e-3, (l, n, part)
                r0 += rows
        else:
            assert torch.equal(y.view(torch.int32), ya[(l, n)].view(torch.int32)), (l, n)
    a.plan.close()
    b.plan.close()


def test_fused_prefill_matches_unfused(cuda, small_model):
    """Prefill over the stacked q|k and gate|up weights: each part of a stacked output within the GEMM
    tolerance of the separate projection's output, the other projections identical."""
    torch = cuda
    fused = small_model.fused()
    a = decode.PrefillStep(small_model, 64, seed=5)
    b = decode.PrefillStep(fused, 64, seed=5)
    s = torch.cuda.current_stream().cuda_stream
    a.run(s)
    b.run(s)
    torch.cuda.synchronize()
    for name, y in b.outputs.items():
        if name in fused.parts:
            r0 = 0
            for part, rows in fused.parts[name]:
                assert max_rel(y[:, r0:r0 + rows].cpu().numpy(), a.outputs[part].cpu().numpy()) <= 2e-2, (name, part)
                r0 += rows
        else:
            assert max_rel(y.cpu().numpy(), a.outputs[name].cpu().numpy()) <= 1e-6, name


@pytest.mark.parametrize("m", [1, 8])
def test_fused_ops_step(cuda, small_model, m):
    """The decode step with the engine's fused ops (5 launches a layer + the LM head): graph replays
    equal the eager run bit for bit, and the last layer's outputs agree with the oracle -- q|k and v
    against the fp64 product of rmsnorm(x, attn_norm) (ops.cpp:8-13), the SwiGLU activation against
    silu(g) * u of the fp64 gate / up products of rmsnorm(x, ffn_norm) on a slice of its features,
    ffn_down against the fp64 product of that activation, the LM head against rmsnorm(x,
    output_norm)."""
    torch = cuda
    fm = small_model.fused_ops()
    step = decode.FusedDecodeStep(fm, m, seed=40 + m)
    assert step.launches() == 2 * 5 + 1
    s = torch.cuda.current_stream().cuda_stream
    step.run_eager(s)
    torch.cuda.synchronize()
    bufs = lambda: [*step.out.values(), step.h, step.logits]
    ref = [b.clone() for b in bufs()]
    for rep in range(3):
        for b in bufs():
            b.fill_(float("nan"))
        step.replay(s)
        torch.cuda.synchronize()
        for b, r in zip(bufs(), ref):
            assert torch.equal(b.view(torch.int32), r.view(torch.int32)), rep
    x = step.x.cpu().numpy()
    eps = fm.eps
    last = fm.layers[-1]
    norms = fm.norms[-1]
    xa = oracle.rmsnorm(x, norms["attn_norm"].cpu().numpy(), eps)
    xf = oracle.rmsnorm(x, norms["ffn_norm"].cpu().numpy(), eps)

    def rows_of(w, r0, nr):
        rb = qvx.row_bytes(w.type, w.cols)
        return w.data[r0 * rb:(r0 + nr) * rb].cpu().numpy()

    for k, xin in (("wqk", xa), ("wv", xa)):
        w = last[k]
        r0 = (w.rows // 3) & ~15
        got = step.out[k][:, r0:r0 + 48].cpu().numpy()
        assert max_rel(got, oracle.matmul_f64(rows_of(w, r0, 48), w.type, xin, m, 48, w.cols)) <= 1e-3, k
    gu = last["ffn_gateup"]
    j0 = 16 * 37  # features 592 .. 623: gate rows 1184 .., up rows 1200 .. of the interleaved weight
    g = oracle.matmul_f64(rows_of(gu, 2 * j0, 16), gu.type, xf, m, 16, gu.cols)
    u = oracle.matmul_f64(rows_of(gu, 2 * j0 + 16, 16), gu.type, xf, m, 16, gu.cols)
    h_ref = oracle.swiglu(g.astype(np.float32), u.astype(np.float32)).astype(np.float64)
    h = step.h.cpu().numpy()
    bound = 1e-3 * (1.1 * np.abs(g).max() * np.abs(u).max() + np.abs(g).max() * np.abs(u).max())
    assert np.abs(h[:, j0:j0 + 16] - h_ref).max() <= bound
    wd = last["ffn_down"]
    assert max_rel(step.out["ffn_down"][:, :64].cpu().numpy(),
                   oracle.matmul_f64(rows_of(wd, 0, 64), wd.type, h, m, 64, wd.cols)) <= 1e-3
    lm = fm.lm_head
    xo = oracle.rmsnorm(x, fm.output_norm.cpu().numpy(), eps)
    r0 = 64000
    assert max_rel(step.logits[:, r0:r0 + 48].cpu().numpy(),
                   oracle.matmul_f64(rows_of(lm, r0, 48), lm.type, xo, m, 48, lm.cols)) <= 1e-3
    step.plan.close()


def test_separate_ops_step_matches_fused(cuda, small_model):
    """The reference's op sequence as separate launches (OpsDecodeStep, captured into one graph) and
    the fused step compute the same layer: the standalone norm and the fused prologue share one
    canonical sum, so q (the first rows of q|k) and v agree to the GEMV bar, and so do the SwiGLU
    activation and ffn_down."""
    torch = cuda
    m = 2
    fused = decode.FusedDecodeStep(small_model.fused_ops(), m, seed=60)
    ops = decode.OpsDecodeStep(small_model, m, seed=60)
    s = torch.cuda.current_stream().cuda_stream
    fused.run_eager(s)
    ops.capture()
    ops.replay()
    torch.cuda.synchronize()
    d = small_model.layers[0]["wq"].rows
    pairs = [(fused.out["wqk"][:, :d], ops.out["wq"]), (fused.out["wqk"][:, d:], ops.out["wk"]),
             (fused.out["wv"], ops.out["wv"]), (fused.h, ops.h), (fused.out["ffn_down"], ops.out["ffn_down"]),
             (fused.logits, ops.logits)]
    for i, (a, b) in enumerate(pairs):
        assert max_rel(a.cpu().numpy(), b.cpu().numpy().astype(np.float64)) <= 2e-3, i
    fused.plan.close()
