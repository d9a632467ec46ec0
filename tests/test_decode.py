"""CPU tests of the decode-step caller (qorvix_amd/decode.py): the token's GEMV list mirrors the
reference's decoder call order and type mix, its byte accounting is the GGUF arithmetic, and the
plan entry points reject bad handles before touching a device."""
from __future__ import annotations

import qorvix_amd as qvx
from qorvix_amd import decode


def test_layer_call_order_mirrors_reference_decoder():
    # runtime/src/text_model.cpp:146-173: wq, wk, wv, (attention), wo, ffn_gate, ffn_up, ffn_down
    assert [s[0] for s in decode.LAYER_SPECS] == ["wq", "wk", "wv", "wo", "ffn_gate", "ffn_up", "ffn_down"]
    specs = decode.sweep_specs()
    assert len(specs) == 32 * 7 + 1 and specs[-1][1] == "lm_head"
    assert [s[1] for s in specs[:7]] == [s[0] for s in decode.LAYER_SPECS]
    # inputs: q/k/v/gate/up read the normed state, wo the attention output, ffn_down the SwiGLU output
    assert {s[0]: s[4] for s in decode.LAYER_SPECS} == {
        "wq": "xn", "wk": "xn", "wv": "xn", "wo": "attn", "ffn_gate": "xn", "ffn_up": "xn", "ffn_down": "act"}


def test_q4_k_m_type_mix():
    types = {s[0]: s[3] for s in decode.LAYER_SPECS}
    assert types["wv"] == qvx.Q6_K and types["ffn_down"] == qvx.Q6_K and decode.LM_HEAD[3] == qvx.Q6_K
    assert all(types[n] == qvx.Q4_K for n in ("wq", "wk", "wo", "ffn_gate", "ffn_up"))


def test_sweep_byte_accounting():
    # per-tensor bytes from the block formats: rows * (cols / 256) * {144 (Q4_K), 210 (Q6_K)}
    per = {"wq": 4096 * 16 * 144, "wk": 1024 * 16 * 144, "wv": 1024 * 16 * 210, "wo": 4096 * 16 * 144,
           "ffn_gate": 14336 * 16 * 144, "ffn_up": 14336 * 16 * 144, "ffn_down": 4096 * 56 * 210}
    assert per == {"wq": 9437184, "wk": 2359296, "wv": 3440640, "wo": 9437184, "ffn_gate": 33030144,
                   "ffn_up": 33030144, "ffn_down": 48168960}
    layer = sum(per.values())
    assert layer == 138903552
    lm = 128256 * 16 * 210
    wb, ab1 = decode.sweep_bytes(1)
    _, ab8 = decode.sweep_bytes(8)
    assert wb == 32 * layer + lm == 4875853824
    # activations in + outputs out, 4 bytes each, per GEMV and vector
    io = sum(rows + cols for _, _, rows, cols, _, _ in decode.sweep_specs()) * 4
    assert ab1 == wb + io == 4886868992
    assert ab8 == wb + 8 * io == 4963975168


def test_plan_entry_points_reject_null_handles():
    lib = qvx.lib()
    assert lib.qvx_plan_size(None) == 0
    assert lib.qvx_plan_launch(None, None) == qvx.E_NULL
    assert lib.qvx_plan_run_eager(None, None) == qvx.E_NULL
    assert lib.qvx_plan_instantiate(None) == qvx.E_NULL
    assert lib.qvx_plan_add_qmatmul_n(None, None, None, qvx.Q4_K, None, 1, 16, 256) == qvx.E_NULL
    assert lib.qvx_plan_create(None) == qvx.E_NULL
    lib.qvx_plan_destroy(None)
    assert qvx.strerror(qvx.E_STATE).startswith("plan not instantiated")


def test_fused_model_stacks_same_input_pairs():
    """Model.fused stacks q with k and gate with up (same type and row length) row-wise; calls()
    then yields 5 GEMVs per layer in the reference's order, each stacked weight in place of its
    first part, and the bytes of each part sit where its rows do."""
    import torch
    from qorvix_amd import decode
    m = decode.Model()
    for l in range(2):
        layer = {}
        for i, (name, rows, cols, t, _) in enumerate(decode.LAYER_SPECS):
            rows, cols = rows // 256, cols // 16  # small stand-ins keeping the type mix and ratios
            nb = qvx.weight_bytes(t, rows, cols)
            layer[name] = decode.DevWeight(torch.full((nb,), 16 * l + i, dtype=torch.uint8), t, rows, cols)
        m.layers.append(layer)
    m.lm_head = decode.DevWeight(torch.zeros(qvx.weight_bytes(qvx.Q6_K, 8, 256), dtype=torch.uint8), qvx.Q6_K, 8, 256)
    f = m.fused()
    names = [(l, n, src) for l, n, _, src in f.calls()]
    per_layer = [("wqk", "xn"), ("wv", "xn"), ("wo", "attn"), ("ffn_gateup", "xn"), ("ffn_down", "act")]
    assert names == [(l, n, s) for l in range(2) for n, s in per_layer] + [(2, "lm_head", "xn")]
    for l in range(2):
        qk, gu = f.layers[l]["wqk"], f.layers[l]["ffn_gateup"]
        q, k = m.layers[l]["wq"], m.layers[l]["wk"]
        assert (qk.rows, qk.cols, qk.type) == (q.rows + k.rows, q.cols, q.type)
        assert torch.equal(qk.data[:q.data.numel()], q.data) and torch.equal(qk.data[q.data.numel():], k.data)
        assert gu.rows == m.layers[l]["ffn_gate"].rows + m.layers[l]["ffn_up"].rows
        assert f.layers[l]["wv"] is m.layers[l]["wv"]  # Q6_K: not stacked with q/k, shared
    assert f.parts["wqk"] == (("wq", 16), ("wk", 4))
    # the unfused model keeps the reference's 7 calls per layer
    assert [n for l, n, _, _ in m.calls() if l == 0] == [s[0] for s in decode.LAYER_SPECS]


def test_fused_step_refuses_a_model_without_norms():
    """Every launch of FusedDecodeStep folds an RMSNorm into its activations; a model whose GGUF file
    lacks a norm tensor is refused up front (before any device work) instead of running un-normed."""
    import pytest

    m = decode.Model(lm_head=None, norms=[{"attn_norm": object(), "ffn_norm": None}], output_norm=None)
    m.layers.append({})
    with pytest.raises(ValueError, match="ffn_norm of layer 0"):
        decode.FusedDecodeStep(m, 1)
    m.norms = []
    with pytest.raises(ValueError, match="attn_norm of layer 0"):
        decode.FusedDecodeStep(m, 1)
    m.norms = [{"attn_norm": object(), "ffn_norm": object()}]
    m.lm_head = object()
    with pytest.raises(ValueError, match="output_norm"):
        decode.FusedDecodeStep(m, 1)
