"""GPU test of the GGUF path end to end: a file holding quantized tensors of every GEMV format is
mapped, each tensor's raw blocks are uploaded with qvx_gguf_upload, and qvx_qmatmul on the uploaded
weights agrees with the oracle computed from the mapped bytes."""
from __future__ import annotations

import numpy as np
import pytest

import oracle
import qorvix_amd as qvx
from conftest import max_rel
from gguf_build import GgufBuilder
from qorvix_amd.gguf import GgufFile

pytestmark = pytest.mark.gpu

HALF_OFFS = {qvx.Q4_0: [0], qvx.Q8_0: [0], qvx.Q4_K: [0, 2], qvx.Q6_K: [208]}
SPECS = [("blk.0.attn_q.weight", qvx.Q4_K, 96, 512), ("blk.0.attn_v.weight", qvx.Q6_K, 40, 768),
         ("blk.0.ffn_up.weight", qvx.Q8_0, 33, 256), ("output.weight", qvx.Q4_0, 70, 1024)]


def blocks(t, rows, cols, rng):
    bs, bb = qvx.type_traits(t)
    n = rows * cols // bs
    w = rng.integers(0, 256, size=(n, bb), dtype=np.uint8)
    for o in HALF_OFFS[t]:
        h = (np.abs(rng.standard_normal(n)) * 0.01 + 1e-4).astype(np.float16).view(np.uint16)
        w[:, o], w[:, o + 1] = h & 0xFF, h >> 8
    return w.reshape(-1)


def test_gguf_upload_and_qmatmul(cuda, tmp_path):
    rng = np.random.default_rng(11)
    b = GgufBuilder(3).str("general.architecture", "llama").u32("general.alignment", 32)
    data, off, ref = bytearray(), 0, {}
    for name, t, rows, cols in SPECS:
        w = blocks(t, rows, cols, rng)
        b.tensor(name, [cols, rows], t, off)
        ref[name] = w
        data += w.tobytes()
        pad = (-len(data)) % 32
        data += b"\0" * pad
        off = len(data)
    path = tmp_path / "model.gguf"
    path.write_bytes(b.build(32, data=bytes(data)))
    with GgufFile.open(path) as f:
        for name, t, rows, cols in SPECS:
            g = f.tensor(name)
            assert (g.rows, g.cols, g.type_raw) == (rows, cols, t)
            assert np.array_equal(f.tensor_bytes(name), ref[name])
            dw = f.upload(name)
            cuda.cuda.synchronize()
            assert np.array_equal(dw.data.cpu().numpy(), ref[name])
            x = cuda.from_numpy(rng.standard_normal(cols).astype(np.float32)).cuda()
            y = qvx.qmatmul_t(dw.data, t, x, rows, cols)
            cuda.cuda.synchronize()
            want = oracle.matmul_f64(ref[name], t, x.cpu().numpy()[None, :], 1, rows, cols)
            assert max_rel(y.cpu().numpy(), want) <= 1e-3, name
        # a destination smaller than the tensor is refused before any copy
        small = cuda.empty(16, dtype=cuda.uint8, device="cuda")
        i = qvx.lib().qvx_gguf_find_tensor(f._h, b"output.weight")
        assert qvx.lib().qvx_gguf_upload(f._h, i, small.data_ptr(), 16, None) == qvx.E_RANGE


def test_decode_step_from_gguf(cuda, tmp_path):
    """A small Llama-shaped GGUF (2 layers, Q4_K_M-style mix, tied LM head) loads through
    decode.Model.from_gguf and its decode step agrees with the oracle on every projection."""
    from qorvix_amd import decode
    rng = np.random.default_rng(5)
    d, kv, ffn, vocab, L = 512, 128, 768, 1000, 2
    b = (GgufBuilder(3).str("general.architecture", "llama").u32("general.alignment", 32)
         .u32("llama.block_count", L).u32("llama.embedding_length", d).u32("llama.feed_forward_length", ffn)
         .u32("llama.attention.head_count", 8).u32("llama.attention.head_count_kv", 2))
    specs = []
    for l in range(L):
        specs += [(f"blk.{l}.attn_q.weight", qvx.Q4_K, d, d), (f"blk.{l}.attn_k.weight", qvx.Q4_K, kv, d),
                  (f"blk.{l}.attn_v.weight", qvx.Q6_K, kv, d), (f"blk.{l}.attn_output.weight", qvx.Q4_K, d, d),
                  (f"blk.{l}.ffn_gate.weight", qvx.Q4_K, ffn, d), (f"blk.{l}.ffn_up.weight", qvx.Q4_K, ffn, d),
                  (f"blk.{l}.ffn_down.weight", qvx.Q6_K, d, ffn)]
    specs.append(("token_embd.weight", qvx.Q6_K, vocab, d))  # tied: no output.weight
    data, ref = bytearray(), {}
    for name, t, rows, cols in specs:
        w = blocks(t, rows, cols, rng)
        b.tensor(name, [cols, rows], t, len(data))
        ref[name] = (w, t, rows, cols)
        data += w.tobytes() + b"\0" * ((-w.size) % 32)
    path = tmp_path / "llama.gguf"
    path.write_bytes(b.build(32, data=bytes(data)))
    model = decode.Model.from_gguf(path)
    assert len(model.layers) == L and model.lm_head.rows == vocab
    step = decode.DecodeStep(model, 2, seed=4)
    step.replay(cuda.cuda.current_stream().cuda_stream)
    cuda.cuda.synchronize()
    X = {k: v.cpu().numpy() for k, v in step.inputs.items()}
    files = {"wq": "attn_q", "wk": "attn_k", "wv": "attn_v", "wo": "attn_output", "ffn_gate": "ffn_gate",
             "ffn_up": "ffn_up", "ffn_down": "ffn_down"}
    src = {s[0]: s[4] for s in decode.LAYER_SPECS}
    for l, name, y in step.outputs:
        key = f"blk.{l}.{files[name]}.weight" if name in files else "token_embd.weight"
        w, t, rows, cols = ref[key]
        want = oracle.matmul_f64(w, t, X[src.get(name, "xn")], 2, rows, cols)
        assert max_rel(y.cpu().numpy(), want) <= 1e-3, (l, name)
    step.plan.close()
