"""qorvix_amd -- MI355X (gfx950) engine for the QorVix GGUF quantized matmul.

Host-side Python mirror of the reference operator (``runtime/include/qorvix/runtime/qmatmul.hpp``
and ``dequant.hpp``) over the C ABI of ``libqvx.so`` (``include/qvx.h``).  The functions keep the
reference's names, argument meaning and error behaviour: the reference returns ``false`` where
these return ``False`` (or raise, for the ``*_t`` tensor helpers), with the same cases rejected
before any device work.

Two layers:

* raw-pointer functions (``qmatmul``, ``qmatmul_n``, ``dequantize``, ``dequant_row``,
  ``qgemm_f16`` ...) taking device addresses and a HIP stream handle -- the C ABI as is;
* torch helpers (``qmatmul_t`` ...) taking ``torch.Tensor``s on ``cuda`` and launching on the
  current torch stream; PyTorch is only the device-memory and stream plumbing.

There is no CPU fallback: if ``libqvx.so`` is missing or no GPU is present, calls raise.
"""
from __future__ import annotations

import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libqvx.so")

# ggml type ids (public GGUF format)
F32, F16, Q4_0, Q4_1, Q5_0, Q5_1, Q8_0, Q8_1, Q4_K, Q5_K, Q6_K, BF16 = 0, 1, 2, 3, 6, 7, 8, 9, 12, 13, 14, 30
TYPE_NAMES = {0: "F32", 1: "F16", 2: "Q4_0", 3: "Q4_1", 6: "Q5_0", 7: "Q5_1", 8: "Q8_0", 9: "Q8_1",
              12: "Q4_K", 13: "Q5_K", 14: "Q6_K", 30: "BF16"}

# status codes (include/qvx.h)
OK, E_TYPE, E_SHAPE, E_NVEC, E_NULL, E_HIP, E_VARIANT, E_RANGE, E_STATE = 0, -1, -2, -3, -4, -5, -6, -7, -8
E_FORMAT, E_IO, E_LIB = -9, -10, -11
# GEMM variants
GEMM_BF16, GEMM_I8, GEMM_F16 = 0, 1, 2

# The C ABI: name -> (argtypes, restype).  tests/test_capi.py checks this table against qvx.h.
_vp, _u32, _i32, _sz, _u64, _f32 = C.c_void_p, C.c_uint32, C.c_int, C.c_size_t, C.c_uint64, C.c_float
SIGNATURES = {
    "qvx_version": ([], C.c_char_p),
    "qvx_strerror": ([_i32], C.c_char_p),
    "qvx_supports": ([_u32], _i32),
    "qvx_can_dequantize": ([_u32], _i32),
    "qvx_type_traits": ([_u32, C.POINTER(_u32), C.POINTER(_u32)], _i32),
    "qvx_fp16_to_float": ([C.c_uint16], _f32),
    "qvx_bf16_to_float": ([C.c_uint16], _f32),
    "qvx_qmatmul": ([_vp, _vp, _u32, _vp, _i32, _i32, _vp], _i32),
    "qvx_qmatmul_n": ([_vp, _vp, _u32, _vp, _i32, _i32, _i32, _vp], _i32),
    "qvx_qmatmul_n_bias": ([_vp, _vp, _u32, _vp, _vp, _i32, _i32, _i32, _vp], _i32),
    "qvx_qmatmul_n_rmsnorm": ([_vp, _vp, _u32, _vp, _vp, _f32, _i32, _i32, _i32, _vp], _i32),
    "qvx_qmatmul_group": ([_vp, _vp, _vp, _vp, _i32, _vp, _vp, _f32, _i32, _vp], _i32),
    "qvx_qmatmul_swiglu": ([_vp, _vp, _u32, _vp, _vp, _f32, _i32, _i32, _i32, _vp], _i32),
    "qvx_interleave_rows16": ([_vp, _vp, _vp, _u32, _i32, _i32, _vp], _i32),
    "qvx_rmsnorm": ([_vp, _vp, _vp, _f32, _i32, _i32, _vp], _i32),
    "qvx_swiglu": ([_vp, _vp, _vp, _sz, _vp], _i32),
    "qvx_dequantize": ([_u32, _vp, _vp, _sz, _vp], _i32),
    "qvx_dequant_row": ([_vp, _u32, _i32, _i32, _vp, _vp], _i32),
    "qvx_qgemm_f16": ([_vp, _vp, _u32, _vp, _i32, _i32, _i32, _i32, _vp], _i32),
    "qvx_qgemm_f16_noalloc": ([_vp, _vp, _u32, _vp, _i32, _i32, _i32, _i32, _vp], _i32),
    "qvx_qgemm_plan_q4k": ([_i32, _i32, _i32, _i32, _vp, _i32], _i32),
    "qvx_gemm16": ([_vp, _vp, _vp, _i32, _i32, _i32, _i32, _vp], _i32),
    "qvx_dequantize16": ([_u32, _vp, _vp, _sz, _i32, _vp], _i32),
    "qvx_quantize_act_q8": ([_vp, _i32, _i32, _vp, _vp, _vp, _vp], _i32),
    "qvx_fill_synthetic": ([_vp, _u32, _i32, _i32, _u64, _f32, _vp], _i32),
    "qvx_fill_normal_f32": ([_vp, _sz, _u64, _f32, _vp], _i32),
    "qvx_fill_normal_f16": ([_vp, _sz, _u64, _f32, _vp], _i32),
    "qvx_bench_read": ([_vp, _sz, _vp, _vp], _i32),
    "qvx_plan_create": ([C.POINTER(_vp)], _i32),
    "qvx_plan_add_qmatmul_n": ([_vp, _vp, _vp, _u32, _vp, _i32, _i32, _i32], _i32),
    "qvx_plan_add_qmatmul_n_rmsnorm": ([_vp, _vp, _vp, _u32, _vp, _vp, _f32, _i32, _i32, _i32], _i32),
    "qvx_plan_add_qmatmul_swiglu": ([_vp, _vp, _vp, _u32, _vp, _vp, _f32, _i32, _i32, _i32], _i32),
    "qvx_plan_add_qmatmul_group": ([_vp, _vp, _vp, _vp, _vp, _i32, _vp, _vp, _f32, _i32], _i32),
    "qvx_plan_fork": ([_vp], _i32),
    "qvx_plan_join": ([_vp], _i32),
    "qvx_plan_size": ([_vp], _i32),
    "qvx_plan_instantiate": ([_vp], _i32),
    "qvx_plan_launch": ([_vp, _vp], _i32),
    "qvx_plan_run_eager": ([_vp, _vp], _i32),
    "qvx_plan_destroy": ([_vp], None),
    "qvx_gguf_open": ([C.c_char_p, C.POINTER(_vp)], _i32),
    "qvx_gguf_parse": ([_vp, _sz, C.POINTER(_vp)], _i32),
    "qvx_gguf_close": ([_vp], None),
    "qvx_gguf_last_error": ([], C.c_char_p),
    "qvx_gguf_version": ([_vp], _u32),
    "qvx_gguf_alignment": ([_vp], _u32),
    "qvx_gguf_data_offset": ([_vp], _u64),
    "qvx_gguf_tensor_count": ([_vp], C.c_int64),
    "qvx_gguf_meta_count": ([_vp], C.c_int64),
    "qvx_gguf_find_tensor": ([_vp, C.c_char_p], C.c_int64),
    "qvx_gguf_tensor_info": ([_vp, C.c_int64, C.POINTER(C.c_char_p), C.POINTER(_u32), C.POINTER(_u32),
                              C.POINTER(_u64), C.POINTER(_u64), C.POINTER(_u64), C.POINTER(_u64)], _i32),
    "qvx_gguf_tensor_data": ([_vp, C.c_int64], _vp),
    "qvx_gguf_upload": ([_vp, C.c_int64, _vp, _sz, _vp], _i32),
    "qvx_gguf_meta_key": ([_vp, C.c_int64], C.c_char_p),
    "qvx_gguf_meta_type": ([_vp, C.c_char_p, C.POINTER(_u32), C.POINTER(_u32), C.POINTER(_u64)], _i32),
    "qvx_gguf_meta_u64": ([_vp, C.c_char_p, _u64, C.POINTER(_u64)], _i32),
    "qvx_gguf_meta_i64": ([_vp, C.c_char_p, _u64, C.POINTER(C.c_int64)], _i32),
    "qvx_gguf_meta_f64": ([_vp, C.c_char_p, _u64, C.POINTER(C.c_double)], _i32),
    "qvx_gguf_meta_bool": ([_vp, C.c_char_p, _u64, C.POINTER(_i32)], _i32),
    "qvx_gguf_meta_string": ([_vp, C.c_char_p, _u64, C.POINTER(C.c_void_p), C.POINTER(_sz)], _i32),
    "qvx_qmatmul_host": ([_vp, _vp, _u32, _vp, _i32, _i32], _i32),
    "qvx_qmatmul_n_host": ([_vp, _vp, _u32, _vp, _i32, _i32, _i32], _i32),
    "qvx_dequantize_host": ([_u32, _vp, _vp, _sz], _i32),
    "qvx_dequant_row_host": ([_vp, _u32, _i32, _i32, _vp], _i32),
}

_lib = None


class QvxError(RuntimeError):
    """A qvx entry point returned a negative status."""

    def __init__(self, code: int, what: str = ""):
        self.code = code
        super().__init__(f"{what}: qvx status {code} ({strerror(code)})" if what else strerror(code))


def lib():
    """Loads libqvx.so (raises if it was never built: there is no fallback path)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"{LIB_PATH} is missing; run __graft_entry__.build() or "
                              "python qorvix_amd/buildlib.py first")
        so = C.CDLL(LIB_PATH)
        for name, (argtypes, restype) in SIGNATURES.items():
            fn = getattr(so, name)
            fn.argtypes = argtypes
            fn.restype = restype
        _lib = so
    return _lib


def build() -> str:
    """Compile libqvx.so in-tree (hipcc, gfx950) and return its path."""
    from . import buildlib
    global _lib
    _lib = None
    return buildlib.build()


def strerror(code: int) -> str:
    try:
        return lib().qvx_strerror(code).decode()
    except ImportError:
        return f"status {code}"


def version() -> str:
    return lib().qvx_version().decode()


# ---- reference-shaped API (raw device pointers; bool results like the reference) -----------------

def supports(ggml_type: int) -> bool:
    """qmatmulSupports (runtime/src/qmatmul.cpp:24-26) for the GPU kernels."""
    return bool(lib().qvx_supports(ggml_type))


def can_dequantize(ggml_type: int) -> bool:
    """canDequantize (runtime/src/dequant.cpp:257-275)."""
    return bool(lib().qvx_can_dequantize(ggml_type))


def type_traits(ggml_type: int):
    """(block_size, type_size) or None (gguf/src/gguf_types.cpp:49-54)."""
    b, n = C.c_uint32(), C.c_uint32()
    if not lib().qvx_type_traits(ggml_type, C.byref(b), C.byref(n)):
        return None
    return b.value, n.value


def fp16_to_float(h: int) -> float:
    """fp16ToFloat (runtime/src/dequant.cpp:222-248)."""
    return lib().qvx_fp16_to_float(h)


def bf16_to_float(b: int) -> float:
    """bf16ToFloat (runtime/src/dequant.cpp:250-255)."""
    return lib().qvx_bf16_to_float(b)


def row_bytes(ggml_type: int, cols: int) -> int:
    bs, ts = type_traits(ggml_type)
    return cols // bs * ts


def weight_bytes(ggml_type: int, rows: int, cols: int) -> int:
    return rows * row_bytes(ggml_type, cols)


def qmatmul(out: int, weight: int, ggml_type: int, x: int, rows: int, cols: int, stream: int = 0) -> int:
    """out[r] = dot(dequant(row r), x) on device pointers (runtime/src/qmatmul.cpp:28-62). Status."""
    return lib().qvx_qmatmul(out, weight, ggml_type, x, rows, cols, stream)


def qmatmul_n(out: int, weight: int, ggml_type: int, X: int, nvec: int, rows: int, cols: int,
              stream: int = 0) -> int:
    """Batched form (runtime/src/qmatmul.cpp:64-115); out [nvec, rows]. Status."""
    return lib().qvx_qmatmul_n(out, weight, ggml_type, X, nvec, rows, cols, stream)


GROUP_MAX = 8


def qmatmul_group(outs, weights, types, rows, x: int, cols: int, stream: int = 0, norm_w: int = 0,
                  eps: float = 1e-5) -> int:
    """outs[i] = W_i . xn for the members (device pointers; types and row counts per member), xn =
    rmsnorm(x, norm_w, eps) when norm_w else x: the decoder's rmsnorm and q / k / v wmatmuls
    (runtime/src/text_model.cpp:146-149) in one call, each output bit-identical to qmatmul's (or
    qmatmul_n_rmsnorm's). Status."""
    n = len(outs)
    if not (len(weights) == len(types) == len(rows) == n):
        raise ValueError("qmatmul_group: one output, weight, type and row count per member")
    arr = C.c_void_p * max(n, 1)
    return lib().qvx_qmatmul_group(arr(*outs), arr(*weights), (C.c_uint32 * max(n, 1))(*types),
                                   (C.c_int32 * max(n, 1))(*rows), n, x, norm_w or None, eps, cols, stream)


def qmatmul_n_bias(out: int, weight: int, ggml_type: int, X: int, bias: int, nvec: int, rows: int, cols: int,
                   stream: int = 0) -> int:
    """wmatmulNBias (runtime/include/qorvix/runtime/weights.hpp:68-80) on device pointers: the product
    plus bias[rows] (bias 0 = no bias). Status."""
    return lib().qvx_qmatmul_n_bias(out, weight, ggml_type, X, bias, nvec, rows, cols, stream)


def qmatmul_n_rmsnorm(out: int, weight: int, ggml_type: int, X: int, norm_w: int, eps: float, nvec: int, rows: int,
                      cols: int, stream: int = 0) -> int:
    """out = W . rmsnorm(x) per vector: the decoder's ops::rmsnorm + wmatmul
    (runtime/src/text_model.cpp:146-149, ops.cpp:8-13) in one call. Status."""
    return lib().qvx_qmatmul_n_rmsnorm(out, weight, ggml_type, X, norm_w, eps, nvec, rows, cols, stream)


def qmatmul_swiglu(out: int, weight_gu: int, ggml_type: int, X: int, norm_w: int, eps: float, nvec: int, ffn: int,
                   cols: int, stream: int = 0) -> int:
    """out = silu(W_gate . xn) * (W_up . xn), xn = rmsnorm(x) when norm_w (else x), over a gate|up weight
    interleaved in 16-row groups (text_model.cpp:161-165, ops.cpp:96-100). Status."""
    return lib().qvx_qmatmul_swiglu(out, weight_gu, ggml_type, X, norm_w or None, eps, nvec, ffn, cols, stream)


def rmsnorm(out: int, x: int, w: int, eps: float, nvec: int, n: int, stream: int = 0) -> int:
    """ops::rmsnorm (runtime/src/ops.cpp:8-13) over nvec rows of n on device pointers. Status."""
    return lib().qvx_rmsnorm(out, x, w, eps, nvec, n, stream)


def swiglu(out: int, gate: int, up: int, n: int, stream: int = 0) -> int:
    """ops::swiglu (runtime/src/ops.cpp:96-100) on device pointers. Status."""
    return lib().qvx_swiglu(out, gate, up, n, stream)


def dequantize(ggml_type: int, src: int, dst: int, n: int, stream: int = 0) -> int:
    """dequantize (runtime/src/dequant.cpp:277-296) on device pointers. Status."""
    return lib().qvx_dequantize(ggml_type, src, dst, n, stream)


def dequant_row(weight: int, ggml_type: int, cols: int, row: int, dst: int, stream: int = 0) -> int:
    """dequantRow (runtime/src/qmatmul.cpp:117-126) on device pointers. Status."""
    return lib().qvx_dequant_row(weight, ggml_type, cols, row, dst, stream)


def qgemm_f16(out: int, weight: int, ggml_type: int, X: int, M: int, rows: int, cols: int,
              variant: int = GEMM_BF16, stream: int = 0) -> int:
    """Prefill GEMM, X fp16 [M, cols] -> out fp32 [M, rows] on the matrix cores. Status."""
    return lib().qvx_qgemm_f16(out, weight, ggml_type, X, M, rows, cols, variant, stream)


# ---- torch helpers (device tensors, current stream; raise on failure) ------------------------------

def _stream():
    import torch
    return torch.cuda.current_stream().cuda_stream


def _check(rc: int, what: str) -> None:
    if rc != OK:
        raise QvxError(rc, what)


def empty_weight(ggml_type: int, rows: int, cols: int, device="cuda"):
    """A uint8 device tensor sized for a [rows, cols] weight of ggml_type."""
    import torch
    return torch.empty(weight_bytes(ggml_type, rows, cols), dtype=torch.uint8, device=device)


def fill_synthetic_t(w, ggml_type: int, rows: int, cols: int, seed: int, scale_mul: float):
    _check(lib().qvx_fill_synthetic(w.data_ptr(), ggml_type, rows, cols, seed, scale_mul, _stream()),
           "qvx_fill_synthetic")
    return w


def fill_normal_t(x, seed: int, mul: float = 1.0):
    import torch
    if x.dtype == torch.float32:
        _check(lib().qvx_fill_normal_f32(x.data_ptr(), x.numel(), seed, mul, _stream()), "fill_normal_f32")
    elif x.dtype == torch.float16:
        _check(lib().qvx_fill_normal_f16(x.data_ptr(), x.numel(), seed, mul, _stream()), "fill_normal_f16")
    else:
        raise TypeError("fill_normal_t takes float32 or float16 tensors")
    return x


def qmatmul_t(w, ggml_type: int, x, rows: int, cols: int, out=None):
    """out[rows] fp32 = W x for a device weight tensor and fp32 x [cols] (or [n, cols])."""
    import torch
    nvec = 1 if x.dim() == 1 else x.shape[0]
    if out is None:
        out = torch.empty((nvec, rows) if x.dim() > 1 else (rows,), dtype=torch.float32, device=x.device)
    _check(lib().qvx_qmatmul_n(out.data_ptr(), w.data_ptr(), ggml_type, x.data_ptr(), nvec, rows, cols,
                               _stream()), "qvx_qmatmul_n")
    return out


def dequantize_t(w, ggml_type: int, n: int, out=None):
    import torch
    if out is None:
        out = torch.empty(n, dtype=torch.float32, device=w.device)
    _check(lib().qvx_dequantize(ggml_type, w.data_ptr(), out.data_ptr(), n, _stream()), "qvx_dequantize")
    return out


def qgemm_t(w, ggml_type: int, X, rows: int, cols: int, variant: int = GEMM_BF16, out=None):
    import torch
    M = X.shape[0]
    if out is None:
        out = torch.empty((M, rows), dtype=torch.float32, device=X.device)
    _check(lib().qvx_qgemm_f16(out.data_ptr(), w.data_ptr(), ggml_type, X.data_ptr(), M, rows, cols, variant,
                               _stream()), "qvx_qgemm_f16")
    return out


def gemm16_t(X, B, variant: int = GEMM_BF16, out=None):
    """out fp32 [M, N] = X [M, K] . B [N, K]^T for 16-bit device tensors (bf16 or fp16 bits, any
    16-bit dtype): the engine's plain matrix-core GEMM (qvx_gemm16)."""
    import torch
    M, K = X.shape
    N = B.shape[0]
    if out is None:
        out = torch.empty((M, N), dtype=torch.float32, device=X.device)
    _check(lib().qvx_gemm16(out.data_ptr(), X.data_ptr(), B.data_ptr(), M, N, K, variant, _stream()), "qvx_gemm16")
    return out


def dequantize16_t(w, ggml_type: int, n: int, bf16: bool, out=None):
    """The first n elements of a device weight as 16-bit values (qvx_dequantize16): the reference's
    dequantised value rounded once to bf16 (bf16=True) or fp16; an int16 tensor of the bits."""
    import torch
    if out is None:
        out = torch.empty(n, dtype=torch.int16, device=w.device)
    _check(lib().qvx_dequantize16(ggml_type, w.data_ptr(), out.data_ptr(), n, 1 if bf16 else 0, _stream()),
           "qvx_dequantize16")
    return out


def qgemm_plan_q4k(M: int, rows: int, cols: int, cus: int = 0):
    """Launches of the Q4_K bf16 / fp16 GEMM for an M x rows x cols call (qvx_qgemm_plan_q4k): a list
    of dicts with bm, splits, tiles, cols_a, mt_a, base_a, mt_b, base_b.  Host only."""
    desc = (C.c_int * 16)()
    n = lib().qvx_qgemm_plan_q4k(M, rows, cols, cus, desc, 2)
    _check(n if n < 0 else 0, "qvx_qgemm_plan_q4k")
    keys = ("bm", "splits", "tiles", "cols_a", "mt_a", "base_a", "mt_b", "base_b")
    return [dict(zip(keys, desc[8 * i:8 * i + 8])) for i in range(n)]


def rmsnorm_t(x, w, eps: float, out=None):
    """rmsnorm over the last dimension of an fp32 device tensor ([n] or [nvec, n])."""
    import torch
    n = x.shape[-1]
    nvec = x.numel() // n if n else 1
    if out is None:
        out = torch.empty_like(x)
    _check(lib().qvx_rmsnorm(out.data_ptr(), x.data_ptr(), w.data_ptr(), eps, nvec, n, _stream()), "qvx_rmsnorm")
    return out


def swiglu_t(gate, up, out=None):
    import torch
    if out is None:
        out = torch.empty_like(gate)
    _check(lib().qvx_swiglu(out.data_ptr(), gate.data_ptr(), up.data_ptr(), gate.numel(), _stream()), "qvx_swiglu")
    return out


def qmatmul_rmsnorm_t(w, ggml_type: int, x, norm_w, eps: float, rows: int, cols: int, out=None):
    """W . rmsnorm(x) for fp32 x [cols] or [n, cols] (one launch where the kernel folds the norm in)."""
    import torch
    nvec = 1 if x.dim() == 1 else x.shape[0]
    if out is None:
        out = torch.empty((nvec, rows) if x.dim() > 1 else (rows,), dtype=torch.float32, device=x.device)
    _check(lib().qvx_qmatmul_n_rmsnorm(out.data_ptr(), w.data_ptr(), ggml_type, x.data_ptr(), norm_w.data_ptr(), eps,
                                       nvec, rows, cols, _stream()), "qvx_qmatmul_n_rmsnorm")
    return out


def qmatmul_swiglu_t(w_gu, ggml_type: int, x, ffn: int, cols: int, norm_w=None, eps: float = 0.0, out=None):
    """silu(W_gate . xn) * (W_up . xn) for an interleaved gate|up weight (interleave_rows16_t); [ffn] or [n, ffn]."""
    import torch
    nvec = 1 if x.dim() == 1 else x.shape[0]
    if out is None:
        out = torch.empty((nvec, ffn) if x.dim() > 1 else (ffn,), dtype=torch.float32, device=x.device)
    nw = norm_w.data_ptr() if norm_w is not None else None
    _check(lib().qvx_qmatmul_swiglu(out.data_ptr(), w_gu.data_ptr(), ggml_type, x.data_ptr(), nw, eps, nvec, ffn,
                                    cols, _stream()), "qvx_qmatmul_swiglu")
    return out


def interleave_rows16_t(a, b, ggml_type: int, rows: int, cols: int):
    """The gate|up weight qmatmul_swiglu reads: a and b ([rows, cols] raw blocks) in 16-row groups."""
    import torch
    out = torch.empty(2 * weight_bytes(ggml_type, rows, cols), dtype=torch.uint8, device=a.device)
    _check(lib().qvx_interleave_rows16(out.data_ptr(), a.data_ptr(), b.data_ptr(), ggml_type, rows, cols, _stream()),
           "qvx_interleave_rows16")
    return out
