"""ctypes loaders for the CPU checkers.  TEST INFRASTRUCTURE ONLY.

Only tests/, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import this
package, and only to check the HIP engine or to time the CPU operator beside it.  The product
(``qorvix_amd``) never imports it.

* :func:`lib` -- ``liboracle.so``, the plain-C restatement in ``qvx_oracle.c`` of the reference's
  ``runtime/src/dequant.cpp``, ``runtime/src/qmatmul.cpp`` and ``runtime/src/cpu_features.cpp``
  plus the build-defined fp64 and Q8-activation oracles.
* :func:`ref_lib` -- ``_ref/libqvxref.so``, the reference's own CPU operator compiled from its
  sources by ``Makefile`` (absent when the reference tree was never available to build it).
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(HERE, "liboracle.so")
REF_SO = os.path.join(HERE, "_ref", "libqvxref.so")

_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_f64p = np.ctypeslib.ndpointer(np.float64, flags="C_CONTIGUOUS")
_u8p = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")
_i8p = np.ctypeslib.ndpointer(np.int8, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")

_lib = None
_ref = None


def build(force: bool = False) -> None:
    """Compile liboracle.so (and _ref when the reference tree exists) with make."""
    args = ["make", "-s", "-C", HERE, "all"]
    if force:
        args.insert(1, "-B")
    subprocess.run(args, check=True)


def _bind(so, prefix):
    so_fns = {
        "supports": ([C.c_uint32], C.c_int),
        "can_dequantize": ([C.c_uint32], C.c_int),
        "fp16_to_float": ([C.c_uint16], C.c_float),
        "dequantize": ([C.c_uint32, C.c_void_p, _f32p, C.c_size_t], C.c_int),
        "qmatmul": ([_f32p, C.c_void_p, C.c_uint32, _f32p, C.c_int, C.c_int], C.c_int),
        "qmatmul_n": ([_f32p, C.c_void_p, C.c_uint32, _f32p, C.c_int, C.c_int, C.c_int], C.c_int),
        "dequant_row": ([C.c_void_p, C.c_uint32, C.c_int, C.c_int, _f32p], C.c_int),
        "dot_kernel": ([], C.c_char_p),
    }
    for name, (argtypes, restype) in so_fns.items():
        fn = getattr(so, prefix + name)
        fn.argtypes = argtypes
        fn.restype = restype


def _bind_ops(so, prefix):
    f = getattr(so, prefix + "rmsnorm")
    f.argtypes = [_f32p, _f32p, _f32p, C.c_int, C.c_float]
    f.restype = None
    f = getattr(so, prefix + "swiglu")
    f.argtypes = [_f32p, _f32p, _f32p, C.c_int]
    f.restype = None


def lib():
    """The C restatement (liboracle.so), built on first use if missing."""
    global _lib
    if _lib is None:
        if not os.path.exists(ORACLE_SO):
            build()
        so = C.CDLL(ORACLE_SO)
        _bind(so, "qvxo_")
        so.qvxo_bf16_to_float.argtypes = [C.c_uint16]
        so.qvxo_bf16_to_float.restype = C.c_float
        so.qvxo_type_traits.argtypes = [C.c_uint32, C.POINTER(C.c_uint32), C.POINTER(C.c_uint32)]
        so.qvxo_type_traits.restype = C.c_int
        so.qvxo_dot_f32.argtypes = [_f32p, _f32p, C.c_int]
        so.qvxo_dot_f32.restype = C.c_float
        so.qvxo_k4_scale_min.argtypes = [C.c_int, _u8p, C.POINTER(C.c_uint8), C.POINTER(C.c_uint8)]
        so.qvxo_k4_scale_min.restype = None
        so.qvxo_matmul_f64.argtypes = [_f64p, C.c_void_p, C.c_uint32, _f32p, C.c_int, C.c_int, C.c_int]
        so.qvxo_matmul_f64.restype = C.c_int
        so.qvxo_quantize_q8_act.argtypes = [_f32p, C.c_int, C.c_int, _i8p, _f32p, _i32p]
        so.qvxo_quantize_q8_act.restype = None
        _bind_ops(so, "qvxo_")
        _lib = so
    return _lib


def ref_lib():
    """The reference's own CPU operator (oracle/_ref), or None when it was never built."""
    global _ref
    if _ref is None and os.path.exists(REF_SO):
        so = C.CDLL(REF_SO)
        _bind(so, "qvxr_")
        _bind_ops(so, "qvxr_")
        _ref = so
    return _ref


# ---- numpy conveniences ------------------------------------------------------------------------

def _ptr(a: np.ndarray) -> int:
    return a.ctypes.data


def traits(t: int):
    b, n = C.c_uint32(), C.c_uint32()
    if not lib().qvxo_type_traits(t, C.byref(b), C.byref(n)):
        return None
    return b.value, n.value


def dequantize(t: int, blocks: np.ndarray, n: int, use_ref: bool = False) -> np.ndarray:
    out = np.empty(n, np.float32)
    so = ref_lib() if use_ref else lib()
    fn = so.qvxr_dequantize if use_ref else so.qvxo_dequantize
    if not fn(t, _ptr(np.ascontiguousarray(blocks)), out, n):
        raise ValueError(f"type {t} not dequantizable")
    return out


def qmatmul(w: np.ndarray, t: int, x: np.ndarray, rows: int, cols: int, use_ref: bool = False):
    out = np.zeros(rows, np.float32)
    so = ref_lib() if use_ref else lib()
    fn = so.qvxr_qmatmul if use_ref else so.qvxo_qmatmul
    ok = fn(out, _ptr(np.ascontiguousarray(w)), t, np.ascontiguousarray(x, np.float32), rows, cols)
    return out if ok else None


def qmatmul_n(w: np.ndarray, t: int, X: np.ndarray, nvec: int, rows: int, cols: int,
              use_ref: bool = False):
    out = np.zeros(max(nvec, 1) * rows, np.float32)
    so = ref_lib() if use_ref else lib()
    fn = so.qvxr_qmatmul_n if use_ref else so.qvxo_qmatmul_n
    ok = fn(out, _ptr(np.ascontiguousarray(w)), t, np.ascontiguousarray(X, np.float32), nvec, rows, cols)
    return out.reshape(max(nvec, 1), rows) if ok else None


def matmul_f64(w: np.ndarray, t: int, X: np.ndarray, nvec: int, rows: int, cols: int) -> np.ndarray:
    out = np.zeros(nvec * rows, np.float64)
    ok = lib().qvxo_matmul_f64(out, _ptr(np.ascontiguousarray(w)), t,
                               np.ascontiguousarray(X, np.float32), nvec, rows, cols)
    if not ok:
        raise ValueError("matmul_f64 rejected its arguments")
    return out.reshape(nvec, rows)


def quantize_q8_act(X: np.ndarray):
    X = np.ascontiguousarray(X, np.float32)
    M, K = X.shape
    q = np.empty((M, K), np.int8)
    s = np.empty((M, K // 32), np.float32)
    qs = np.empty((M, K // 32), np.int32)
    lib().qvxo_quantize_q8_act(X, M, K, q, s, qs)
    return q, s, qs


def dequant_row(w: np.ndarray, t: int, cols: int, row: int, use_ref: bool = False):
    out = np.zeros(cols, np.float32)
    so = ref_lib() if use_ref else lib()
    fn = so.qvxr_dequant_row if use_ref else so.qvxo_dequant_row
    ok = fn(_ptr(np.ascontiguousarray(w)), t, cols, row, out)
    return out if ok else None


def rmsnorm(x: np.ndarray, w: np.ndarray, eps: float, use_ref: bool = False) -> np.ndarray:
    """The reference's ops::rmsnorm over each row of x (restated, or the reference build)."""
    x = np.ascontiguousarray(np.atleast_2d(x), np.float32)
    w = np.ascontiguousarray(w, np.float32)
    so = ref_lib() if use_ref else lib()
    fn = so.qvxr_rmsnorm if use_ref else so.qvxo_rmsnorm
    out = np.empty_like(x)
    for v in range(x.shape[0]):
        row = np.empty(x.shape[1], np.float32)
        fn(row, np.ascontiguousarray(x[v]), w, x.shape[1], eps)
        out[v] = row
    return out


def swiglu(gate: np.ndarray, up: np.ndarray, use_ref: bool = False) -> np.ndarray:
    """The reference's ops::swiglu, elementwise over equal-shaped arrays."""
    g = np.ascontiguousarray(gate, np.float32).ravel()
    u = np.ascontiguousarray(up, np.float32).ravel()
    so = ref_lib() if use_ref else lib()
    fn = so.qvxr_swiglu if use_ref else so.qvxo_swiglu
    out = np.empty_like(g)
    fn(out, g, u, g.size)
    return out.reshape(np.shape(gate))
