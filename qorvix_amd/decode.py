"""Decode-step caller of the quantized matmul: the weight side of one Llama token.

Mirrors the reference's decoder (``runtime/src/text_model.cpp:146-173``): per layer, ``wmatmul`` of
wq, wk, wv on the normed hidden state, wo on the attention output, ffn_gate and ffn_up on the normed
state, ffn_down on the SwiGLU activation, then the LM head (``:176-177``).  ``wmatmul`` dispatches
on the weight's ggml type (``runtime/include/qorvix/runtime/weights.hpp:49-56``; on the GPU, the
type switch of ``cuda/src/cuda_backend.cu:1523-1542``), which here is ``qvx_qmatmul_n``: the
engine's kernels pick the format.  A token's projections are recorded into a ``Plan`` (one HIP
graph, ``qvx_plan_*`` in ``include/qvx.h``) and replayed with one launch, as the CUDA backend
replays its captured decode step.

``DecodeStep`` issues only the matmuls: RMSNorm, RoPE, attention and SwiGLU are outside it, so their
outputs are stand-in activation buffers (seeded N(0,1)) of the right shapes.  This is the
"full-model decode weight sweep" workload: 32 layers x 7 projections + the LM head = 225 GEMVs and
4,875,853,824 weight bytes per token for Llama-3-8B Q4_K_M.

``FusedDecodeStep`` runs the same weights with the decoder ops the engine owns folded into the
GEMVs (``qvx_qmatmul_n_rmsnorm``, ``qvx_qmatmul_swiglu``): per layer q|k and v on rmsnorm(x,
attn_norm), o on the attention output, gate|up on rmsnorm(x, ffn_norm) with the SwiGLU epilogue,
down on that SwiGLU output, and the LM head on rmsnorm(x, output_norm) -- 5 launches a layer.  RoPE,
attention and the residual adds stay outside, so the hidden state x and the attention output are
stand-ins; the FFN's SwiGLU activation is the engine's own.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass, field

from . import (F32, GEMM_F16, OK, Q4_K, Q6_K, QvxError, empty_weight, fill_normal_t, fill_synthetic_t, lib,
               weight_bytes)


@dataclass
class DevWeight:
    """A device-resident GGUF weight [rows, cols] of one ggml type (``cuda_backend.cu:1257-1262``,
    ``DevWeight``; the quantized case of ``WeightMat``, ``weights.hpp:22-46``)."""
    data: object          # torch.uint8 tensor on the device, raw GGUF blocks row-major
    type: int
    rows: int
    cols: int

    @property
    def nbytes(self) -> int:
        return weight_bytes(self.type, self.rows, self.cols)


def wmatmul_n(out, w: DevWeight, X, nvec: int, stream: int) -> None:
    """out[nvec, rows] = X[nvec, cols] W^T (``weights.hpp:68-87``, ``wmatmulN`` without bias)."""
    rc = lib().qvx_qmatmul_n(out.data_ptr(), w.data.data_ptr(), w.type, X.data_ptr(), nvec, w.rows, w.cols,
                             stream)
    if rc != OK:
        raise QvxError(rc, "qvx_qmatmul_n")


# Llama-3-8B projection shapes (rows = out features, cols = in features) and the Q4_K_M type mix:
# attn_v and ffn_down in Q6_K, the rest Q4_K.
D_MODEL, D_FF, D_KV, VOCAB, N_LAYERS = 4096, 14336, 1024, 128256, 32
LAYER_SPECS = (  # (name, rows, cols, type, input buffer)
    ("wq", D_MODEL, D_MODEL, Q4_K, "xn"),
    ("wk", D_KV, D_MODEL, Q4_K, "xn"),
    ("wv", D_KV, D_MODEL, Q6_K, "xn"),
    ("wo", D_MODEL, D_MODEL, Q4_K, "attn"),
    ("ffn_gate", D_FF, D_MODEL, Q4_K, "xn"),
    ("ffn_up", D_FF, D_MODEL, Q4_K, "xn"),
    ("ffn_down", D_MODEL, D_FF, Q6_K, "act"),
)
LM_HEAD = ("lm_head", VOCAB, D_MODEL, Q6_K, "xn")
INPUTS = {spec[0]: spec[4] for spec in LAYER_SPECS}

# Projections of one type and row length that read the same input, stacked row-wise into one weight
# so that one GEMV computes both (rows are independent, so each row's arithmetic is a one-weight
# call's under the stacked launch geometry): q with k (attn_v is Q6_K in Q4_K_M files), gate with up.
FUSED = (("wqk", ("wq", "wk")), ("ffn_gateup", ("ffn_gate", "ffn_up")))


def sweep_specs(n_layers: int = N_LAYERS, lm_head: bool = True):
    """The (layer, name, rows, cols, type, input) list of one token, in the reference's call order."""
    out = [(l, *spec) for l in range(n_layers) for spec in LAYER_SPECS]
    if lm_head:
        out.append((n_layers, *LM_HEAD))
    return out


def sweep_bytes(m: int, n_layers: int = N_LAYERS, lm_head: bool = True):
    """(weight bytes, algorithmic bytes) per token at M vectors: weights + 4 M (rows + cols) per GEMV."""
    wb = ab = 0
    for _, _, rows, cols, t, _ in sweep_specs(n_layers, lm_head):
        w = weight_bytes(t, rows, cols)
        wb += w
        ab += w + 4 * m * (rows + cols)
    return wb, ab


NORM_EPS = 1e-5  # Llama-3 rms_norm_eps (the GGUF key llama.attention.layer_norm_rms_epsilon)


@dataclass
class Model:
    """Synthetic Llama-3-8B Q4_K_M weights on the device (``layers[l][name]``, ``lm_head``) and the
    RMSNorm weights (``norms[l]`` = {"attn_norm", "ffn_norm"} fp32 [d], ``output_norm``)."""
    layers: list = field(default_factory=list)
    lm_head: DevWeight | None = None
    # name of a stacked weight -> ((part name, rows), ...) in row order (see FUSED)
    parts: dict = field(default_factory=dict)
    norms: list = field(default_factory=list)
    output_norm: object = None
    eps: float = NORM_EPS

    def fused(self) -> "Model":
        """The same weights with each FUSED pair of a layer stacked into one device weight when the
        two share type and row length (the other projections are shared, not copied)."""
        import torch
        m = Model(lm_head=self.lm_head, norms=self.norms, output_norm=self.output_norm, eps=self.eps)
        for layer in self.layers:
            out, used = {}, set()
            for name, (a, b) in FUSED:
                wa, wb = layer.get(a), layer.get(b)
                if wa is None or wb is None or wa.type != wb.type or wa.cols != wb.cols:
                    continue
                out[name] = DevWeight(torch.cat([wa.data, wb.data]), wa.type, wa.rows + wb.rows, wa.cols)
                m.parts[name] = ((a, wa.rows), (b, wb.rows))
                used.update((a, b))
            out.update({k: w for k, w in layer.items() if k not in used})
            m.layers.append(out)
        return m

    def fused_ops(self) -> "Model":
        """The weights as FusedDecodeStep reads them: q and k stacked (as ``fused``), gate and up
        interleaved in 16-row groups (``qvx_interleave_rows16``, the layout of the SwiGLU epilogue),
        the rest shared."""
        import torch
        from . import interleave_rows16_t
        m = Model(lm_head=self.lm_head, norms=self.norms, output_norm=self.output_norm, eps=self.eps)
        for layer in self.layers:
            out = {k: w for k, w in layer.items() if k not in ("wq", "wk", "ffn_gate", "ffn_up")}
            wq, wk, wg, wu = layer["wq"], layer["wk"], layer["ffn_gate"], layer["ffn_up"]
            if wq.type == wk.type and wq.cols == wk.cols:
                out["wqk"] = DevWeight(torch.cat([wq.data, wk.data]), wq.type, wq.rows + wk.rows, wq.cols)
            else:
                out["wq"], out["wk"] = wq, wk
            if wg.type != wu.type or wg.rows != wu.rows or wg.cols != wu.cols or wg.rows % 16:
                raise ValueError("gate and up must share type and shape (rows a multiple of 16) to interleave")
            out["ffn_gateup"] = DevWeight(interleave_rows16_t(wg.data, wu.data, wg.type, wg.rows, wg.cols), wg.type,
                                          2 * wg.rows, wg.cols)
            m.layers.append(out)
        return m

    def calls(self):
        """(layer, name, weight, input) per GEMV of one token: the reference's order
        (text_model.cpp:146-177), a stacked weight taking the place of its first part."""
        for l, layer in enumerate(self.layers):
            first = {parts[0][0]: name for name, parts in self.parts.items() if name in layer}
            skip = {p[0] for name, parts in self.parts.items() if name in layer for p in parts[1:]}
            for name, *_ in LAYER_SPECS:
                if name in skip:
                    continue
                key = first.get(name, name)
                yield l, key, layer[key], INPUTS[name]
        if self.lm_head is not None:
            yield len(self.layers), LM_HEAD[0], self.lm_head, LM_HEAD[4]

    @staticmethod
    def synthetic(n_layers: int = N_LAYERS, lm_head: bool = True, seed: int = 5, device="cuda") -> "Model":
        """Fresh seed per (layer, tensor); scales fp16(|N(0,1)| * 1e-3) as the configs specify."""
        import torch
        m = Model()
        for l in range(n_layers):
            m.norms.append({k: _norm_weight(D_MODEL, _tensor_seed(seed, l, k), device) for k in ("attn_norm", "ffn_norm")})
        m.output_norm = _norm_weight(D_MODEL, _tensor_seed(seed, n_layers, "output_norm"), device)
        for l, name, rows, cols, t, _ in sweep_specs(n_layers, lm_head):
            w = DevWeight(empty_weight(t, rows, cols, device), t, rows, cols)
            fill_synthetic_t(w.data, t, rows, cols, seed=_tensor_seed(seed, l, name), scale_mul=1e-3)
            if l < n_layers:
                while len(m.layers) <= l:
                    m.layers.append({})
                m.layers[l][name] = w
            else:
                m.lm_head = w
        return m

    @staticmethod
    def from_gguf(file, device="cuda") -> "Model":
        """A Llama-family model's matmul weights from a GGUF file (a path or a gguf.GgufFile), by
        the reference's tensor names and checks (runtime/src/weights.cpp:20-50; loadMat,
        runtime/include/qorvix/runtime/tensor_load.hpp:51-63): each projection must exist, hold
        rows x cols elements and have a type the engine computes; the LM head is output.weight, or
        token_embd.weight when the file ties them (weights.hpp:119, lmHead()).  The raw blocks are
        uploaded once and kept quantized."""
        from . import supports
        from .gguf import GgufFile
        f = file if isinstance(file, GgufFile) else GgufFile.open(file)
        n_layers = f.arch_u64("block_count")
        if n_layers is None:
            raise ValueError(f"GGUF file has no {f.architecture or '<arch>'}.block_count")
        d = f.arch_u64("embedding_length")
        ffn = f.arch_u64("feed_forward_length")
        heads, kv_heads = f.arch_u64("attention.head_count"), f.arch_u64("attention.head_count_kv")
        kv = d * (kv_heads or heads) // heads if d and heads else None

        def load(name, rows, cols):
            t = f.tensor(name)
            if t is None:
                raise ValueError(f"missing tensor '{name}'")
            rows = t.rows if rows is None else rows
            cols = t.cols if cols is None else cols
            if t.n_elements != rows * cols:
                raise ValueError(f"tensor '{name}' has {t.n_elements} elements, expected {rows} x {cols}")
            if not supports(t.type_raw):
                raise ValueError(f"tensor '{name}' uses unsupported type {t.type_name()}")
            return f.upload(name, device)

        m = Model()
        shapes = {"wq": (d, d), "wk": (kv, d), "wv": (kv, d), "wo": (d, d), "ffn_gate": (ffn, d),
                  "ffn_up": (ffn, d), "ffn_down": (d, ffn)}
        names = {"wq": "attn_q", "wk": "attn_k", "wv": "attn_v", "wo": "attn_output", "ffn_gate": "ffn_gate",
                 "ffn_up": "ffn_up", "ffn_down": "ffn_down"}
        def load_norm(name):
            t = f.tensor(name)
            if t is None:
                return None
            if t.type_raw != F32 or t.n_elements != d:
                raise ValueError(f"norm tensor '{name}' must be F32 with {d} elements")
            import torch
            return f.upload(name, device).data.view(torch.float32)

        for layer in range(n_layers):
            m.layers.append({k: load(f"blk.{layer}.{names[k]}.weight", *shapes[k]) for k, *_ in LAYER_SPECS})
            m.norms.append({"attn_norm": load_norm(f"blk.{layer}.attn_norm.weight"),
                            "ffn_norm": load_norm(f"blk.{layer}.ffn_norm.weight")})
        head = "output.weight" if f.tensor("output.weight") is not None else "token_embd.weight"
        m.lm_head = load(head, None, d)
        m.output_norm = load_norm("output_norm.weight")
        eps = f.get_f64(f"{f.architecture}.attention.layer_norm_rms_epsilon") if f.architecture else None
        m.eps = float(eps) if eps is not None else NORM_EPS
        return m

    @property
    def nbytes(self) -> int:
        n = sum(w.nbytes for layer in self.layers for w in layer.values())
        return n + (self.lm_head.nbytes if self.lm_head else 0)


def _input_widths(model: Model) -> dict:
    """Row length of each activation buffer (xn, attn, act), from the first layer's calls."""
    return {src: w.cols for l, _, w, src in model.calls() if l == 0}


def _tensor_seed(seed: int, layer: int, name: str) -> int:
    names = [s[0] for s in LAYER_SPECS] + [LM_HEAD[0], "attn_norm", "ffn_norm", "output_norm"]
    return (seed << 20) + (layer << 4) + names.index(name)


def _norm_weight(n: int, seed: int, device):
    """A synthetic RMSNorm weight: 1 + 0.1 N(0,1) (trained Llama norm weights sit around 1)."""
    import torch
    w = torch.empty(n, dtype=torch.float32, device=device)
    fill_normal_t(w, seed=seed, mul=0.1)
    return w.add_(1.0)


class Plan:
    """A recorded GEMV sequence replayed as one HIP graph (``qvx_plan_*``)."""

    def __init__(self):
        h = C.c_void_p()
        rc = lib().qvx_plan_create(C.byref(h))
        if rc != OK:
            raise QvxError(rc, "qvx_plan_create")
        self._h = h

    def add(self, out, w: DevWeight, X, nvec: int) -> None:
        rc = lib().qvx_plan_add_qmatmul_n(self._h, out.data_ptr(), w.data.data_ptr(), w.type, X.data_ptr(), nvec,
                                          w.rows, w.cols)
        if rc != OK:
            raise QvxError(rc, "qvx_plan_add_qmatmul_n")

    def add_rmsnorm(self, out, w: DevWeight, X, norm_w, eps: float, nvec: int) -> None:
        """out = W . rmsnorm(X) (``qvx_plan_add_qmatmul_n_rmsnorm``)."""
        rc = lib().qvx_plan_add_qmatmul_n_rmsnorm(self._h, out.data_ptr(), w.data.data_ptr(), w.type, X.data_ptr(),
                                                  norm_w.data_ptr(), eps, nvec, w.rows, w.cols)
        if rc != OK:
            raise QvxError(rc, "qvx_plan_add_qmatmul_n_rmsnorm")

    def add_swiglu(self, out, w_gu: DevWeight, X, norm_w, eps: float, nvec: int) -> None:
        """out = silu(W_gate . xn) * (W_up . xn) over an interleaved gate|up weight
        (``qvx_plan_add_qmatmul_swiglu``; xn = rmsnorm(X) when norm_w is given)."""
        nw = norm_w.data_ptr() if norm_w is not None else None
        rc = lib().qvx_plan_add_qmatmul_swiglu(self._h, out.data_ptr(), w_gu.data.data_ptr(), w_gu.type,
                                               X.data_ptr(), nw, eps, nvec, w_gu.rows // 2, w_gu.cols)
        if rc != OK:
            raise QvxError(rc, "qvx_plan_add_qmatmul_swiglu")

    def add_group(self, outs, ws, X, norm_w=None, eps: float = 1e-5) -> None:
        """outs[i] = ws[i] . xn for one vector X, xn = rmsnorm(X, norm_w, eps) when norm_w is given
        else X, as one grouped call (``qvx_plan_add_qmatmul_group``)."""
        n = len(ws)
        arr = C.c_void_p * n
        nw = norm_w.data_ptr() if norm_w is not None else None
        rc = lib().qvx_plan_add_qmatmul_group(self._h, arr(*[o.data_ptr() for o in outs]),
                                              arr(*[w.data.data_ptr() for w in ws]),
                                              (C.c_uint32 * n)(*[w.type for w in ws]),
                                              (C.c_int32 * n)(*[w.rows for w in ws]), n, X.data_ptr(), nw, eps,
                                              ws[0].cols)
        if rc != OK:
            raise QvxError(rc, "qvx_plan_add_qmatmul_group")

    def fork(self) -> None:
        rc = lib().qvx_plan_fork(self._h)
        if rc != OK:
            raise QvxError(rc, "qvx_plan_fork")

    def join(self) -> None:
        rc = lib().qvx_plan_join(self._h)
        if rc != OK:
            raise QvxError(rc, "qvx_plan_join")

    def __len__(self) -> int:
        return lib().qvx_plan_size(self._h)

    def instantiate(self) -> None:
        rc = lib().qvx_plan_instantiate(self._h)
        if rc != OK:
            raise QvxError(rc, "qvx_plan_instantiate")

    def launch(self, stream: int) -> None:
        rc = lib().qvx_plan_launch(self._h, stream)
        if rc != OK:
            raise QvxError(rc, "qvx_plan_launch")

    def run_eager(self, stream: int) -> None:
        rc = lib().qvx_plan_run_eager(self._h, stream)
        if rc != OK:
            raise QvxError(rc, "qvx_plan_run_eager")

    def close(self) -> None:
        if self._h:
            lib().qvx_plan_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class DecodeStep:
    """The weight side of one decode step at M vectors: activation stand-ins, per-projection
    outputs, and the plan of 7 GEMVs per layer + the LM head in the reference's order."""

    def __init__(self, model: Model, m: int, seed: int = 9, device="cuda", concurrent: bool = False,
                 grouped: bool = False):
        import torch
        if concurrent and model.parts:
            raise ValueError("concurrent q/k/v and gate/up branches are for the unfused model")
        if grouped and (concurrent or m != 1):
            raise ValueError("grouped calls take one vector, in order")
        self.model, self.m = model, m
        f32 = dict(dtype=torch.float32, device=device)
        self.inputs = {k: torch.empty((m, c), **f32) for k, c in _input_widths(model).items()}
        for i, k in enumerate(("xn", "attn", "act")):
            fill_normal_t(self.inputs[k], seed=seed + i)
        self.outputs = []
        self.plan = Plan()
        pending = []  # grouped: the q/k/v or gate/up members collected so far
        for l, name, w, src in model.calls():
            y = torch.empty((m, w.rows), **f32)
            self.outputs.append((l, name, y))
            if grouped and name in ("wq", "wk", "wqk", "wv", "ffn_gate", "ffn_up"):
                # q/k/v read the same normed state (q|k stacked or not), and so do gate/up when they
                # are not stacked: one grouped launch each
                pending.append((y, w))
                if name in ("wv", "ffn_up"):
                    self.plan.add_group([o for o, _ in pending], [x for _, x in pending], self.inputs[src])
                    pending = []
                continue
            # ... or independent graph branches when asked (measured slower on MI355X: the graph's
            # cross-branch joins cost more than the overlap)
            if concurrent and name in ("wq", "ffn_gate"):
                self.plan.fork()
            self.plan.add(y, w, self.inputs[src], m)
            if concurrent and name in ("wv", "ffn_up"):
                self.plan.join()
        self.plan.instantiate()

    def replay(self, stream: int) -> None:
        self.plan.launch(stream)

    def run_eager(self, stream: int) -> None:
        self.plan.run_eager(stream)


class FusedDecodeStep:
    """One decode step at M vectors with the engine's fused decoder ops (5 launches a layer + the LM
    head; 4 with ``grouped``, q|k and v then sharing one launch at M = 1), in the reference's order (text_model.cpp:146-177) on a ``Model.fused_ops()`` model:
    per layer qk = Wqk . rmsnorm(x, attn_norm) and v = Wv . rmsnorm(x, attn_norm) (text_model.cpp:
    146-149), o = Wo . attn (:158), h = swiglu(Wgate . xn, Wup . xn) with xn = rmsnorm(x, ffn_norm)
    (:161-165), down = Wdown . h (:166); logits = Wlm . rmsnorm(x, output_norm) (:171-172).  x (the
    residual stream) and attn (the attention output) are seeded stand-ins, h is the SwiGLU output
    the step itself computes; one output buffer per projection, reused across layers."""

    def __init__(self, model: Model, m: int, seed: int = 9, device="cuda", grouped: bool = False):
        import torch
        # every fused launch folds a norm into its activations: refuse a model without them rather than
        # run the projections on un-normed inputs
        for l in range(len(model.layers)):
            for k in ("attn_norm", "ffn_norm"):
                if l >= len(model.norms) or model.norms[l].get(k) is None:
                    raise ValueError(f"FusedDecodeStep needs {k} of layer {l}; the model has none")
        if model.lm_head is not None and model.output_norm is None:
            raise ValueError("FusedDecodeStep needs output_norm for the LM head; the model has none")
        if grouped and m != 1:
            raise ValueError("grouped calls take one vector")
        self.model, self.m = model, m
        f32 = dict(dtype=torch.float32, device=device)
        l0 = model.layers[0]
        d = l0["wo"].rows
        self.x = fill_normal_t(torch.empty((m, d), **f32), seed=seed)
        self.attn = fill_normal_t(torch.empty((m, l0["wo"].cols), **f32), seed=seed + 1)
        self.out = {k: torch.empty((m, w.rows), **f32) for k, w in l0.items() if k != "ffn_gateup"}
        self.h = torch.empty((m, l0["ffn_gateup"].rows // 2), **f32)
        self.logits = torch.empty((m, model.lm_head.rows), **f32) if model.lm_head is not None else None
        self.plan = Plan()
        eps = model.eps
        for l, layer in enumerate(model.layers):
            an, fn = model.norms[l]["attn_norm"], model.norms[l]["ffn_norm"]
            qkv = [k for k in ("wqk", "wq", "wk", "wv") if k in layer]
            if grouped:  # q|k and v on the normed state in one launch (4 launches a layer)
                self.plan.add_group([self.out[k] for k in qkv], [layer[k] for k in qkv], self.x, an, eps)
            for k in qkv if not grouped else ():
                self.plan.add_rmsnorm(self.out[k], layer[k], self.x, an, eps, m)
            self.plan.add(self.out["wo"], layer["wo"], self.attn, m)
            self.plan.add_swiglu(self.h, layer["ffn_gateup"], self.x, fn, eps, m)
            self.plan.add(self.out["ffn_down"], layer["ffn_down"], self.h, m)
        if model.lm_head is not None:
            self.plan.add_rmsnorm(self.logits, model.lm_head, self.x, model.output_norm, eps, m)
        self.plan.instantiate()

    def launches(self) -> int:
        return len(self.plan)

    def replay(self, stream: int) -> None:
        self.plan.launch(stream)

    def run_eager(self, stream: int) -> None:
        self.plan.run_eager(stream)


class OpsDecodeStep:
    """The same decode step as FusedDecodeStep issued as the reference's op sequence, one launch per
    op (text_model.cpp:146-177): per layer rmsnorm, wq, wk, wv, wo, rmsnorm, ffn_gate, ffn_up, swiglu,
    ffn_down (10 launches) and rmsnorm + the LM head -- the engine's standalone qvx_rmsnorm /
    qvx_swiglu beside the plain GEMVs, on a plain (unstacked) model.  ``capture`` records it into one
    graph (torch.cuda.CUDAGraph; nothing allocates), the baseline the fused step is measured against."""

    def __init__(self, model: Model, m: int, seed: int = 9, device="cuda"):
        import torch
        self.model, self.m = model, m
        f32 = dict(dtype=torch.float32, device=device)
        l0 = model.layers[0]
        d = l0["wo"].rows
        self.x = fill_normal_t(torch.empty((m, d), **f32), seed=seed)
        self.attn = fill_normal_t(torch.empty((m, l0["wo"].cols), **f32), seed=seed + 1)
        self.xn = torch.empty((m, d), **f32)
        self.out = {k: torch.empty((m, w.rows), **f32) for k, w in l0.items()}
        self.h = torch.empty((m, l0["ffn_gate"].rows), **f32)
        self.logits = torch.empty((m, model.lm_head.rows), **f32) if model.lm_head is not None else None
        self.graph = None

    def run(self, stream: int) -> None:
        from . import _check
        so, m, eps = lib(), self.m, self.model.eps

        def norm(w):
            _check(so.qvx_rmsnorm(self.xn.data_ptr(), self.x.data_ptr(), w.data_ptr(), eps, m, self.x.shape[1],
                                  stream), "qvx_rmsnorm")

        for l, layer in enumerate(self.model.layers):
            norm(self.model.norms[l]["attn_norm"])
            for k in ("wq", "wk", "wv"):
                wmatmul_n(self.out[k], layer[k], self.xn, m, stream)
            wmatmul_n(self.out["wo"], layer["wo"], self.attn, m, stream)
            norm(self.model.norms[l]["ffn_norm"])
            wmatmul_n(self.out["ffn_gate"], layer["ffn_gate"], self.xn, m, stream)
            wmatmul_n(self.out["ffn_up"], layer["ffn_up"], self.xn, m, stream)
            _check(so.qvx_swiglu(self.h.data_ptr(), self.out["ffn_gate"].data_ptr(), self.out["ffn_up"].data_ptr(),
                                 self.h.numel(), stream), "qvx_swiglu")
            wmatmul_n(self.out["ffn_down"], layer["ffn_down"], self.h, m, stream)
        if self.model.lm_head is not None:
            norm(self.model.output_norm)
            wmatmul_n(self.logits, self.model.lm_head, self.xn, m, stream)

    def capture(self) -> None:
        import torch
        self.run(torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            self.run(torch.cuda.current_stream().cuda_stream)

    def replay(self, stream: int = 0) -> None:
        self.graph.replay()


def wgemm(out, w: DevWeight, X16, m: int, stream: int, variant: int = GEMM_F16, noalloc: bool = False) -> None:
    """out[m, rows] = X16[m, cols] W^T with X in fp16: the prefill GEMM (``qvx_qgemm_f16``, or
    ``qvx_qgemm_f16_noalloc`` when ``noalloc``: no device allocation, for graph capture)."""
    name = "qvx_qgemm_f16_noalloc" if noalloc else "qvx_qgemm_f16"
    rc = getattr(lib(), name)(out.data_ptr(), w.data.data_ptr(), w.type, X16.data_ptr(), m, w.rows, w.cols, variant,
                              stream)
    if rc != OK:
        raise QvxError(rc, name)


class PrefillStep:
    """The weight side of a prompt prefill of M positions, batched.  The reference prefills token
    by token, one ``forward`` per prompt position (``runtime/src/generator.cpp:24-28``), each
    running the decoder's seven projections per layer; here every projection of a layer takes all M
    positions at once as one GEMM (``qvx_qgemm_f16``: Q4_K on the engine's raw-block MFMA kernels,
    the Q6_K tensors on its dequantising MFMA kernel), and the LM head runs on the last position
    only, as the reference keeps only the logits after the last prompt token.  Activations are
    seeded fp16 stand-ins (norms, RoPE, attention and SwiGLU are outside the engine); one output
    buffer per projection name is reused across layers.  ``run`` issues the calls eagerly;
    ``capture`` records them into one graph through the no-allocation entry point and ``replay``
    launches it."""

    def __init__(self, model: Model, m: int, seed: int = 11, device="cuda", variant: int = GEMM_F16):
        import torch
        self.model, self.m, self.variant = model, m, variant
        f16 = dict(dtype=torch.float16, device=device)
        f32 = dict(dtype=torch.float32, device=device)
        widths = _input_widths(model)
        self.inputs = {k: torch.empty((m, c), **f16) for k, c in widths.items()}
        for i, k in enumerate(("xn", "attn", "act")):
            fill_normal_t(self.inputs[k], seed=seed + i, mul=0.5)
        self.calls = [c for c in model.calls() if c[0] < len(model.layers)]
        self.outputs = {name: torch.empty((m, w.rows), **f32) for l, name, w, _ in self.calls if l == 0}
        self.last = torch.empty((1, widths["xn"]), **f32)  # the last position's normed state
        fill_normal_t(self.last, seed=seed + 3)
        self.logits = torch.empty((1, model.lm_head.rows), **f32) if model.lm_head is not None else None

    def flops(self) -> int:
        """2 * rows * cols per position per layer projection, and once for the LM head."""
        n = sum(2 * self.m * w.rows * w.cols for layer in self.model.layers for w in layer.values())
        if self.model.lm_head is not None:
            n += 2 * self.model.lm_head.rows * self.model.lm_head.cols
        return n

    def run(self, stream: int, noalloc: bool = False) -> None:
        for _, name, w, src in self.calls:
            wgemm(self.outputs[name], w, self.inputs[src], self.m, stream, self.variant, noalloc)
        if self.model.lm_head is not None:
            wmatmul_n(self.logits, self.model.lm_head, self.last, 1, stream)

    def capture(self) -> None:
        """Record the step into a graph (``torch.cuda.CUDAGraph``), every GEMM through
        ``qvx_qgemm_f16_noalloc``.  One eager run first sets up the kernels' launch configuration
        and the device's scratch array outside the capture."""
        import torch
        self.run(torch.cuda.current_stream().cuda_stream, noalloc=True)
        torch.cuda.synchronize()
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            self.run(torch.cuda.current_stream().cuda_stream, noalloc=True)

    def replay(self) -> None:
        self.graph.replay()

