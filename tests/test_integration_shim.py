"""The reference-side binding (qorvix_amd/bindings/qmatmul_qvx.cpp) against the reference's own
headers: it compiles as C++23 with the declarations of runtime/include/qorvix/runtime/qmatmul.hpp
and dequant.hpp (so the signatures line up), and a program that calls the reference's functions
through it, linked with libqvx.so, gets the engine's answers for the calls that need no device --
type predicates, fp16 / bf16 conversion, and every argument rejection (qmatmul.cpp's `false` cases).
Needs the reference sources (present where the engine is built, not on the GPU box) and g++."""
from __future__ import annotations

import os
import shutil
import subprocess

import pytest

import qorvix_amd as qvx

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF_INC = "/root/reference/runtime/include"
SHIM = os.path.join(REPO, "qorvix_amd", "bindings", "qmatmul_qvx.cpp")

pytestmark = pytest.mark.skipif(not os.path.isdir(REF_INC) or shutil.which("g++") is None,
                                reason="needs the reference's headers and g++")

MAIN = r"""
#include <cstdio>
#include <cstring>
#include "qorvix/runtime/dequant.hpp"
#include "qorvix/runtime/qmatmul.hpp"
using namespace qorvix::runtime;
int main() {
  float out[4] = {7, 7, 7, 7}, x[256] = {}, dst[256];
  unsigned char w[1024] = {};
  int bad = 0;
  bad += !qmatmulSupports(12) + !qmatmulSupports(14) + !qmatmulSupports(8) + !qmatmulSupports(2);
  bad += qmatmulSupports(10) + qmatmulSupports(39);         // Q2_K, an unknown id
  bad += !canDequantize(0) + canDequantize(10);
  bad += fp16ToFloat(0x3C00) != 1.0f;                        // 1.0
  bad += fp16ToFloat(0xC000) != -2.0f;
  bad += fp16ToFloat(0x0001) != 5.9604644775390625e-08f;    // smallest subnormal
  bad += bf16ToFloat(0x3F80) != 1.0f;
  bad += bf16ToFloat(0xC2F7) != -123.5f;
  bad += qmatmul(out, w, 10, x, 4, 256);                     // unsupported type
  bad += qmatmul(out, w, 12, x, 4, 300);                     // cols not whole blocks
  bad += qmatmulN(out, w, 12, x, 0, 4, 256);                 // nVec <= 0
  bad += qmatmulN(out, w, 12, x, 1, 4, 100);
  bad += dequantRow(w, 10, 256, 0, dst);
  bad += dequantRow(w, 8, 33, 0, dst);
  bad += dequantize(10, w, dst, 256);
  for (float v : out) bad += v != 7.0f;                      // out untouched on failure
  std::printf("bad=%d\n", bad);
  return bad;
}
"""


def _lib_dir():
    return os.path.dirname(qvx.LIB_PATH)


def test_shim_compiles_against_reference_headers():
    r = subprocess.run(["g++", "-std=c++2b", "-fsyntax-only", "-Wall", "-Wextra", "-Werror", "-I", REF_INC,
                        "-I", os.path.join(REPO, "include"), SHIM], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr


def test_reference_calls_through_shim(tmp_path):
    main = tmp_path / "main.cpp"
    main.write_text(MAIN)
    exe = tmp_path / "shim_main"
    libdir = _lib_dir()
    r = subprocess.run(["g++", "-std=c++2b", "-O1", "-I", REF_INC, "-I", os.path.join(REPO, "include"), str(main), SHIM,
                        "-L", libdir, "-l:libqvx.so", f"-Wl,-rpath,{libdir}", "-o", str(exe)],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    run = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert run.returncode == 0, run.stdout + run.stderr
    assert "bad=0" in run.stdout
