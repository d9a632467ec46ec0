"""CPU tests of the C ABI (libqvx.so): it loads, exports exactly what include/qvx.h declares, and
its host-side logic (type table, fp16 decode, argument checks) behaves like the reference's
operator -- all without touching a GPU (every call here returns before any device work)."""
from __future__ import annotations

import ctypes as C
import os
import re

import numpy as np
import pytest

import qorvix_amd as qvx
from conftest import ROOT

HEADER = os.path.join(ROOT, "include", "qvx.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(qvx_\w+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = qvx.lib()
    names = declared_functions()
    assert len(names) >= 19
    for name in names:
        assert hasattr(lib, name), f"{name} declared in qvx.h but not exported"
    # the Python binding table covers the header exactly
    assert sorted(qvx.SIGNATURES) == names


def test_nm_exports_match_header():
    import subprocess
    out = subprocess.run(["nm", "-D", "--defined-only", qvx.LIB_PATH], capture_output=True, text=True).stdout
    exported = sorted(set(re.findall(r" T (qvx_\w+)", out)))
    assert exported == declared_functions()


def test_no_undefined_engine_symbols():
    """Every kernel's launch stub is defined: a kernel whose stub the host pass dropped (a target
    builtin called from a lambda does that) leaves an undefined qvx:: symbol that fails the load."""
    import subprocess
    out = subprocess.run(["nm", "-D", "--undefined-only", qvx.LIB_PATH], capture_output=True, text=True).stdout
    assert not [ln for ln in out.splitlines() if "3qvx" in ln], out


def test_library_loads_beside_torchs_hip_runtime():
    """The library loads in a process whose HIP runtime is the one torch bundles (the GPU tests'
    setup): every versioned HIP symbol it imports must exist there, which a call new to a later ROCm
    (e.g. an API tagged hip_7.1) would break on the GPU box."""
    import subprocess
    import sys
    code = ("import torch, ctypes, sys; sys.path.insert(0, %r); import qorvix_amd as q; "
            "ctypes.CDLL(q.LIB_PATH); print('ok')" % ROOT)
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=600)
    assert r.returncode == 0 and r.stdout.strip().endswith("ok"), r.stderr[-2000:]


def test_version_and_errors():
    assert "gfx950" in qvx.version()
    assert qvx.strerror(qvx.E_TYPE).startswith("unsupported")
    assert qvx.strerror(qvx.OK) == "ok"
    assert "library" in qvx.strerror(qvx.E_LIB)


def test_type_table_matches_gguf():
    assert qvx.type_traits(qvx.Q4_K) == (256, 144)
    assert qvx.type_traits(qvx.Q6_K) == (256, 210)
    assert qvx.type_traits(qvx.Q8_0) == (32, 34)
    assert qvx.type_traits(qvx.Q4_0) == (32, 18)
    assert qvx.type_traits(4) is None
    # every type the reference's qmatmulSupports accepts (canDequantize && traits)
    for t in (qvx.Q8_0, qvx.Q4_0, qvx.Q4_K, qvx.Q6_K, qvx.F32, qvx.F16, qvx.BF16, qvx.Q4_1, qvx.Q5_0, qvx.Q5_1,
              qvx.Q8_1, qvx.Q5_K):
        assert qvx.supports(t)
    for t in (10, 11, 15, 16, 99):
        assert not qvx.supports(t)
    for t in (0, 1, 2, 3, 6, 7, 8, 9, 12, 13, 14, 30):
        assert qvx.can_dequantize(t)
    assert not qvx.can_dequantize(10)


def test_fp16_to_float_host_all_finite():
    bits = np.arange(65536, dtype=np.uint16)
    finite = bits[(bits & 0x7C00) != 0x7C00]
    got = np.array([qvx.fp16_to_float(int(h)) for h in finite], np.float32)
    np.testing.assert_array_equal(got, finite.view(np.float16).astype(np.float32))


# Argument checks: the reference's false cases (runtime/src/qmatmul.cpp:30-33, :66, :70-72) as codes.
FAKE = 0x1000  # never dereferenced: every call below is rejected (or is a no-op) before device work


def test_qmatmul_rejections():
    lib = qvx.lib()
    assert lib.qvx_qmatmul(FAKE, FAKE, qvx.Q8_0, FAKE, 1, 30, None) == qvx.E_SHAPE  # cols % 32
    assert lib.qvx_qmatmul(FAKE, FAKE, qvx.Q4_K, FAKE, 1, 300, None) == qvx.E_SHAPE  # cols % 256
    assert lib.qvx_qmatmul(FAKE, FAKE, 10, FAKE, 1, 256, None) == qvx.E_TYPE  # Q2_K
    assert lib.qvx_qmatmul(FAKE, FAKE, 4, FAKE, 1, 256, None) == qvx.E_TYPE  # retired id
    assert lib.qvx_qmatmul(FAKE, FAKE, 11, FAKE, 1, 256, None) == qvx.E_TYPE  # Q3_K: not dequantisable
    assert lib.qvx_qmatmul(FAKE, FAKE, qvx.Q5_K, FAKE, 1, 128, None) == qvx.E_SHAPE  # cols % 256
    assert lib.qvx_qgemm_f16(FAKE, FAKE, qvx.F16, FAKE, 128, 256, 256, qvx.GEMM_I8, None) == qvx.E_TYPE  # int8: Q4_K only
    assert lib.qvx_qgemm_f16(FAKE, FAKE, 11, FAKE, 128, 256, 256, qvx.GEMM_F16, None) == qvx.E_TYPE  # Q3_K
    assert lib.qvx_qmatmul_n(FAKE, FAKE, qvx.Q8_0, FAKE, 0, 1, 32, None) == qvx.E_NVEC
    assert lib.qvx_qmatmul_n(FAKE, FAKE, qvx.Q8_0, FAKE, -3, 1, 32, None) == qvx.E_NVEC
    # nVec is checked first, as in the reference (qmatmulN returns false before the type check)
    assert lib.qvx_qmatmul_n(FAKE, FAKE, 10, FAKE, 0, 1, 32, None) == qvx.E_NVEC
    # rows <= 0: nothing to compute, success without touching memory
    assert lib.qvx_qmatmul(FAKE, FAKE, qvx.Q4_K, FAKE, 0, 4096, None) == qvx.OK
    assert lib.qvx_qmatmul(FAKE, FAKE, qvx.Q4_K, FAKE, -5, 4096, None) == qvx.OK
    # null pointers with real work
    assert lib.qvx_qmatmul(None, FAKE, qvx.Q4_K, FAKE, 4, 256, None) == qvx.E_NULL
    assert lib.qvx_qmatmul(FAKE, None, qvx.Q4_K, FAKE, 4, 256, None) == qvx.E_NULL
    assert lib.qvx_qmatmul(FAKE, FAKE, qvx.Q4_K, None, 4, 256, None) == qvx.E_NULL


def test_qmatmul_group_rejections():
    lib = qvx.lib()
    arr = C.c_void_p * 3
    outs, ws = arr(FAKE, FAKE, FAKE), arr(FAKE, FAKE, FAKE)
    types = (C.c_uint32 * 3)(qvx.Q4_K, qvx.Q4_K, qvx.Q6_K)
    rows = (C.c_int32 * 3)(16, 16, 16)
    assert lib.qvx_qmatmul_group(outs, ws, types, rows, 0, FAKE, None, 1e-5, 256, None) == qvx.E_NVEC
    assert lib.qvx_qmatmul_group(outs, ws, types, rows, qvx.GROUP_MAX + 1, FAKE, None, 1e-5, 256, None) == qvx.E_NVEC
    assert lib.qvx_qmatmul_group(None, ws, types, rows, 3, FAKE, None, 1e-5, 256, None) == qvx.E_NULL
    assert lib.qvx_qmatmul_group(outs, ws, types, rows, 3, None, None, 1e-5, 256, None) == qvx.E_NULL
    assert lib.qvx_qmatmul_group(outs, ws, types, rows, 3, FAKE, None, 1e-5, 300, None) == qvx.E_SHAPE  # cols % 256
    bad = (C.c_uint32 * 3)(qvx.Q4_K, 10, qvx.Q6_K)  # Q2_K
    assert lib.qvx_qmatmul_group(outs, ws, bad, rows, 3, FAKE, None, 1e-5, 256, None) == qvx.E_TYPE
    nulls = arr(FAKE, None, FAKE)
    assert lib.qvx_qmatmul_group(outs, nulls, types, rows, 3, FAKE, None, 1e-5, 256, None) == qvx.E_NULL
    # members without rows compute nothing: all empty is a successful no-op
    # a norm with no members to compute is checked no further
    none = (C.c_int32 * 3)(0, -1, 0)
    assert lib.qvx_qmatmul_group(outs, nulls, types, none, 3, FAKE, None, 1e-5, 256, None) == qvx.OK


def test_gemm_and_dequant_rejections():
    lib = qvx.lib()
    assert lib.qvx_qgemm_f16(FAKE, FAKE, qvx.Q4_K, FAKE, 128, 256, 256, 7, None) == qvx.E_VARIANT
    assert lib.qvx_qgemm_f16(FAKE, FAKE, qvx.Q4_K, FAKE, 0, 256, 256, 0, None) == qvx.E_NVEC
    assert lib.qvx_qgemm_f16(FAKE, FAKE, qvx.Q4_K, FAKE, 128, 256, 300, 0, None) == qvx.E_SHAPE
    assert lib.qvx_qgemm_f16(FAKE, FAKE, qvx.Q6_K, FAKE, 128, 256, 256, qvx.GEMM_I8, None) == qvx.E_TYPE
    assert lib.qvx_qgemm_f16(FAKE, FAKE, qvx.Q6_K, FAKE, 128, 256, 300, qvx.GEMM_F16, None) == qvx.E_SHAPE
    assert lib.qvx_qgemm_f16(FAKE, FAKE, qvx.Q6_K, FAKE, 128, 0, 256, qvx.GEMM_F16, None) == qvx.OK  # no rows
    assert lib.qvx_qgemm_f16(None, FAKE, qvx.Q6_K, FAKE, 128, 4, 256, qvx.GEMM_F16, None) == qvx.E_NULL
    # fewer elements than one block: no whole block to convert, a successful no-op (dequant.cpp:124)
    assert lib.qvx_dequantize(qvx.Q4_K, FAKE, FAKE, 100, None) == qvx.OK
    assert lib.qvx_dequantize(qvx.Q4_K, None, FAKE, 300, None) == qvx.E_NULL  # one whole block
    assert lib.qvx_dequantize(10, FAKE, FAKE, 256, None) == qvx.E_TYPE
    assert lib.qvx_dequantize(qvx.Q4_K, FAKE, FAKE, 0, None) == qvx.OK
    # the no-allocation GEMM: the same checks (every type runs on the engine's own kernels, so only
    # the int8 variant of a type other than Q4_K is refused by type)
    assert lib.qvx_qgemm_f16_noalloc(FAKE, FAKE, qvx.Q4_K, FAKE, 128, 256, 256, 7, None) == qvx.E_VARIANT
    assert lib.qvx_qgemm_f16_noalloc(FAKE, FAKE, qvx.Q4_K, FAKE, 0, 256, 256, 0, None) == qvx.E_NVEC
    assert lib.qvx_qgemm_f16_noalloc(FAKE, FAKE, qvx.Q4_K, FAKE, 128, 256, 300, 0, None) == qvx.E_SHAPE
    assert lib.qvx_qgemm_f16_noalloc(FAKE, FAKE, qvx.Q6_K, FAKE, 128, 256, 256, qvx.GEMM_I8, None) == qvx.E_TYPE
    assert lib.qvx_qgemm_f16_noalloc(FAKE, FAKE, 10, FAKE, 128, 256, 256, qvx.GEMM_F16, None) == qvx.E_TYPE
    assert lib.qvx_qgemm_f16_noalloc(FAKE, FAKE, qvx.Q4_K, FAKE, 128, 0, 256, qvx.GEMM_F16, None) == qvx.OK
    assert lib.qvx_qgemm_f16_noalloc(None, FAKE, qvx.Q4_K, FAKE, 128, 4, 256, qvx.GEMM_F16, None) == qvx.E_NULL
    # qvx_qmatmul_n_bias: qvx_qmatmul_n's checks (wmatmulNBias = qmatmulN + the bias add)
    assert lib.qvx_qmatmul_n_bias(FAKE, FAKE, qvx.Q4_K, FAKE, FAKE, 0, 4, 256, None) == qvx.E_NVEC
    assert lib.qvx_qmatmul_n_bias(FAKE, FAKE, qvx.Q4_K, FAKE, FAKE, 2, 4, 300, None) == qvx.E_SHAPE
    assert lib.qvx_qmatmul_n_bias(FAKE, FAKE, 10, FAKE, FAKE, 2, 4, 256, None) == qvx.E_TYPE
    assert lib.qvx_qmatmul_n_bias(FAKE, FAKE, qvx.Q4_K, FAKE, FAKE, 2, 0, 256, None) == qvx.OK
    assert lib.qvx_qmatmul_n_bias(None, FAKE, qvx.Q4_K, FAKE, FAKE, 2, 4, 256, None) == qvx.E_NULL
    assert lib.qvx_gemm16(FAKE, FAKE, FAKE, 4, 4, 64, qvx.GEMM_I8, None) == qvx.E_VARIANT
    assert lib.qvx_gemm16(FAKE, FAKE, FAKE, -1, 4, 64, qvx.GEMM_BF16, None) == qvx.E_SHAPE
    assert lib.qvx_gemm16(FAKE, FAKE, FAKE, 0, 4, 64, qvx.GEMM_BF16, None) == qvx.OK
    assert lib.qvx_gemm16(None, FAKE, FAKE, 4, 4, 64, qvx.GEMM_BF16, None) == qvx.E_NULL
    assert lib.qvx_gemm16(FAKE, None, FAKE, 4, 4, 64, qvx.GEMM_F16, None) == qvx.E_NULL
    assert lib.qvx_dequantize16(10, FAKE, FAKE, 256, 1, None) == qvx.E_TYPE
    assert lib.qvx_dequantize16(qvx.Q4_K, FAKE, FAKE, 100, 1, None) == qvx.OK  # no whole block
    assert lib.qvx_dequantize16(qvx.Q4_K, None, FAKE, 256, 0, None) == qvx.E_NULL
    assert lib.qvx_dequant_row(FAKE, qvx.Q8_0, 32, -1, FAKE, None) == qvx.E_RANGE
    assert lib.qvx_dequant_row(FAKE, qvx.Q8_0, 33, 0, FAKE, None) == qvx.E_SHAPE
    assert lib.qvx_quantize_act_q8(FAKE, 4, 33, FAKE, FAKE, FAKE, None) == qvx.E_SHAPE
    assert lib.qvx_fill_synthetic(FAKE, qvx.F16, 4, 32, 1, 1.0, None) == qvx.E_TYPE


def test_host_entry_points_reject_like_reference():
    lib = qvx.lib()
    out = np.zeros(4, np.float32)
    x = np.ones(64, np.float32)
    w = np.zeros(68, np.uint8)
    p = lambda a: a.ctypes.data
    assert lib.qvx_qmatmul_host(p(out), p(w), qvx.Q8_0, p(x), 1, 30) == qvx.E_SHAPE
    assert lib.qvx_qmatmul_n_host(p(out), p(w), qvx.Q8_0, p(x), 0, 1, 32) == qvx.E_NVEC
    assert lib.qvx_qmatmul_host(p(out), p(w), 10, p(x), 1, 256) == qvx.E_TYPE
    # cols == 0 writes zeros on the host without a device (the reference's empty loop)
    out[:] = 7
    assert lib.qvx_qmatmul_host(p(out), p(w), qvx.Q8_0, p(x), 4, 0) == qvx.OK
    assert np.all(out == 0)
    out[:] = 7  # n below one block: nothing converted, nothing written (the reference's floor)
    assert lib.qvx_dequantize_host(qvx.Q4_K, p(w), p(out), 3) == qvx.OK
    assert np.all(out == 7)
    assert qvx.bf16_to_float(0x3F80) == 1.0 and qvx.bf16_to_float(0xC040) == -3.0


def test_bf16_to_float_all_encodings():
    """bf16ToFloat (dequant.cpp:250-255) for all 65536 encodings: the bits shifted into the high half.
    NaN encodings only as NaN (ctypes widens the float return to a Python double, which quiets
    signalling NaNs)."""
    lib = qvx.lib()
    got = np.array([lib.qvx_bf16_to_float(b) for b in range(65536)], np.float32)
    want = (np.arange(65536, dtype=np.uint32) << 16).view(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    np.testing.assert_array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_product_has_no_cpu_fallback(monkeypatch):
    """Without libqvx.so the product raises instead of computing anywhere else."""
    monkeypatch.setattr(qvx, "_lib", None)
    monkeypatch.setattr(qvx, "LIB_PATH", "/nonexistent/libqvx.so")
    with pytest.raises(ImportError):
        qvx.lib()


def test_product_never_imports_oracle():
    src = os.path.join(ROOT, "qorvix_amd")
    for dirpath, _, files in os.walk(src):
        for f in files:
            if f.endswith((".py", ".hip", ".hpp", ".cpp", ".h")):
                text = open(os.path.join(dirpath, f)).read()
                assert "import oracle" not in text and "liboracle" not in text and "qvxo_" not in text, f


def test_bench_read_rejections():
    lib = qvx.lib()
    assert lib.qvx_bench_read(FAKE, 100, FAKE, None) == qvx.E_RANGE  # not whole 16-byte words
    assert lib.qvx_bench_read(None, 256, FAKE, None) == qvx.E_NULL
    assert lib.qvx_bench_read(FAKE, 256, None, None) == qvx.E_NULL
    assert lib.qvx_bench_read(FAKE + 4, 256, FAKE, None) == qvx.E_RANGE  # source not 16-byte aligned
