"""Writes the known-answer fixtures under tests/golden/ (run in the build container).

Inputs are restatements, in our own code, of the deterministic cases the reference's own tests
use for this path; expected outputs come from the reference's own CPU operator compiled from its
sources (oracle/_ref, built by oracle/Makefile), so the fixtures pin our oracle and our GPU
kernels to the reference's actual results:

  kat_dequant_*.npz   tests/dequant_test.cpp:24-135 cases (one per TEST_CASE block)
  kat_qmatmul_*.npz   tests/qmatmul_test.cpp:41-168 cases
  kat_selftest_*.npz  the CUDA self-test patterns with their double-precision host references
                      (cuda/src/cuda_backend.cu:551-573 Q8_0 64x256, :721-748 Q4_K 32x256,
                      :793-825 Q6_K 32x256, :2368-2404 Q4_K 64x1024)
  rand_*.npz          seeded random blocks per type with the reference's dequant and qmatmul output

Each fixture stores the weight bytes, activations, expected fp32 outputs and, for qmatmul, the
dot kernel the reference dispatched to (bit-exact comparisons require the same one).
"""
from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

import oracle  # noqa: E402  (test infrastructure)

Q4_0, Q4_1, Q5_0, Q8_0, Q4_K, Q6_K, F16, BF16 = 2, 3, 6, 8, 12, 14, 1, 30


def h(v: float) -> int:
    """fp16 bits of v, round to nearest even (as __float2half)."""
    return int(np.array([v], np.float16).view(np.uint16)[0])


def hb(bits: int) -> float:
    return float(np.array([bits], np.uint16).view(np.float16)[0])


def put_half(buf: bytearray, off: int, bits: int) -> None:
    buf[off] = bits & 0xFF
    buf[off + 1] = bits >> 8


# ---- dequant_test.cpp cases -----------------------------------------------------------------------

def kat_dequant():
    cases = {}
    # Q8_0 d = 0.5, qs = 0..31 (dequant_test.cpp:33-42)
    b = bytearray(34)
    put_half(b, 0, 0x3800)
    for i in range(32):
        b[2 + i] = i
    cases["q8_0_pos"] = (Q8_0, bytes(b), 32)
    # Q8_0 negative quants, d = 1 (:44-51)
    b = bytearray(34)
    put_half(b, 0, 0x3C00)
    for i in range(32):
        b[2 + i] = (-i) & 0xFF
    cases["q8_0_neg"] = (Q8_0, bytes(b), 32)
    # Q4_0 split-nibble order, bytes 0x80 (:53-63)
    b = bytearray(18)
    put_half(b, 0, 0x3C00)
    for i in range(16):
        b[2 + i] = 0x80
    cases["q4_0_split"] = (Q4_0, bytes(b), 32)
    # Q4_1 d = 2, m = 0.5, bytes 0x31 (:65-75)
    b = bytearray(20)
    put_half(b, 0, 0x4000)
    put_half(b, 2, 0x3800)
    for i in range(16):
        b[4 + i] = 0x31
    cases["q4_1"] = (Q4_1, bytes(b), 32)
    # Q5_0 5th bit (:77-94), both qh states
    b = bytearray(22)
    put_half(b, 0, 0x3C00)
    cases["q5_0_qh0"] = (Q5_0, bytes(b), 32)
    b[2] = 0x01
    cases["q5_0_qh1"] = (Q5_0, bytes(b), 32)
    # Q6_K uniform block, then ql[0] = 0x0F (:96-110)
    b = bytearray(210)
    for i in range(16):
        b[192 + i] = 1
    put_half(b, 208, 0x3C00)
    cases["q6_k_uniform"] = (Q6_K, bytes(b), 256)
    b[0] = 0x0F
    cases["q6_k_one"] = (Q6_K, bytes(b), 256)
    # Q4_K uniform scales, then qs[0] = 5 (:112-128)
    b = bytearray(144)
    put_half(b, 0, 0x3C00)
    for i in range(12):
        b[4 + i] = 1
    cases["q4_k_uniform"] = (Q4_K, bytes(b), 256)
    b[16] = 0x05
    cases["q4_k_one"] = (Q4_K, bytes(b), 256)
    # fp16 / bf16 known encodings (:24-31)
    cases["f16_known"] = (F16, np.array([0x3C00, 0x3800, 0x0000, 0xC000], np.uint16).tobytes(), 4)
    cases["bf16_known"] = (BF16, np.array([0x3F80, 0x4040], np.uint16).tobytes(), 2)
    return cases


# ---- qmatmul_test.cpp cases ---------------------------------------------------------------------

def q8_block(d_bits: int, base: int) -> bytes:
    b = bytearray(34)
    put_half(b, 0, d_bits)
    for i in range(32):
        b[2 + i] = (base + i) & 0xFF
    return bytes(b)


def q8_weight(rows: int, blocks: int) -> bytes:
    scales = [0x3800, 0x3C00, 0x3400, 0x3E00]  # qmatmul_test.cpp:104-111
    return b"".join(q8_block(scales[(r + b) % 4], r * 3 + b) for r in range(rows) for b in range(blocks))


def kat_qmatmul():
    cases = {}
    # Q8_0 3x64 (qmatmul_test.cpp:41-56)
    w = b"".join(q8_block(0x3800, r * 2) + q8_block(0x3C00, r * 2 + 1) for r in range(3))
    x = np.array([0.1 * ((i % 5) - 2) for i in range(64)], np.float32)
    cases["q8_0_3x64"] = (Q8_0, w, x[None, :], 3, 64)
    # Q4_K 2x256 (:58-77)
    rows = []
    for r in range(2):
        b = bytearray(144)
        b[1] = 0x3C
        for i in range(12):
            b[4 + i] = 1
        for i in range(128):
            b[16 + i] = (r + i) & 0x0F
        rows.append(bytes(b))
    x = np.array([0.01 * ((i % 7) - 3) for i in range(256)], np.float32)
    cases["q4_k_2x256"] = (Q4_K, b"".join(rows), x[None, :], 2, 256)
    # qmatmulN bit-identity 12x64 x 5 vectors (:114-135)
    X = np.array([0.01 * (i % 23) - 0.1 for i in range(5 * 64)], np.float32).reshape(5, 64)
    cases["q8_0_n5"] = (Q8_0, q8_weight(12, 2), X, 12, 64)
    # more vectors than the 64-wide tile: 4x32 x 70 (:137-156)
    X = np.array([(i % 7) * 0.05 for i in range(70 * 32)], np.float32).reshape(70, 32)
    cases["q8_0_n70"] = (Q8_0, q8_weight(4, 1), X, 4, 32)
    # one vector (:158-168)
    cases["q8_0_n1"] = (Q8_0, q8_weight(3, 1), np.full((1, 32), 0.25, np.float32), 3, 32)
    return cases


# ---- CUDA self-test patterns (deterministic bytes + double-precision references) ---------------------

def k4_scale_min(j, q):
    if j < 4:
        return q[j] & 63, q[j + 4] & 63
    return (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4), (q[j + 4] >> 4) | ((q[j] >> 6) << 4)


def q4k_fill(seed: int) -> bytes:
    b = bytearray(144)
    put_half(b, 0, h(np.float32(0.02) * np.float32(seed % 5 + 1)))
    put_half(b, 2, h(np.float32(0.01)))
    for i in range(12):
        b[4 + i] = (seed * 3 + i * 5) & 0x3F
    for i in range(128):
        b[16 + i] = (seed + i) & 0xFF
    return bytes(b)


def q4k_ref_f64(blk: bytes, x: np.ndarray) -> float:
    d = hb(blk[0] | blk[1] << 8)
    dmin = hb(blk[2] | blk[3] << 8)
    sc_bytes = blk[4:16]
    qs = blk[16:144]
    acc = 0.0
    for i in range(256):
        s, chunk, local = i // 32, i // 64, i % 64
        qb = qs[chunk * 32 + (local & 31)]
        nib = (qb & 0xF) if local < 32 else (qb >> 4)
        sc, m = k4_scale_min(s, sc_bytes)
        acc += (d * sc * nib - dmin * m) * float(x[i])
    return acc


def selftests():
    cases = {}
    # Q8_0 64x256 (cuda_backend.cu:551-573)
    rows, cols = 64, 256
    x = np.array([np.float32(0.1) * np.float32((i % 5) - 2) for i in range(cols)], np.float32)
    W = bytearray()
    ref = np.zeros(rows)
    for r in range(rows):
        acc = 0.0
        for b in range(cols // 32):
            hs = h(np.float32(0.02) * np.float32((r % 7) + 1))
            blk = bytearray(34)
            put_half(blk, 0, hs)
            d = hb(hs)
            for i in range(32):
                q = ((r + b + i) % 15) - 7
                blk[2 + i] = q & 0xFF
                acc += d * float(np.float32(q)) * float(x[b * 32 + i])
            W += blk
        ref[r] = acc
    cases["selftest_q8_0_64x256"] = (Q8_0, bytes(W), x[None, :], rows, cols, ref)
    # Q4_K 32x256 (:721-748)
    x = np.array([np.float32(0.02) * np.float32((i % 9) - 4) for i in range(256)], np.float32)
    blks = [q4k_fill(r) for r in range(32)]
    ref = np.array([q4k_ref_f64(b, x) for b in blks])
    cases["selftest_q4_k_32x256"] = (Q4_K, b"".join(blks), x[None, :], 32, 256, ref)
    # Q6_K 32x256 (:793-825)
    W = bytearray()
    ref = np.zeros(32)
    for r in range(32):
        blk = bytearray(210)
        for i in range(128):
            blk[i] = (r + i) & 0xFF
        for i in range(64):
            blk[128 + i] = (r * 2 + i) & 0xFF
        for i in range(16):
            blk[192 + i] = (((r + i) % 9) - 4) & 0xFF
        put_half(blk, 208, h(np.float32(0.01) * np.float32(r % 4 + 1)))
        d = hb(blk[208] | blk[209] << 8)
        sc = np.array(blk[192:208], np.uint8).view(np.int8)
        acc = 0.0
        for i in range(256):
            half, p = i >> 7, i & 127
            l, quarter, is_ = p & 31, p >> 5, (p & 31) >> 4
            qlh = blk[half * 64:half * 64 + 64]
            qhh = blk[128 + half * 32:128 + half * 32 + 32]
            if quarter == 0:
                lo, hi = qlh[l] & 0xF, qhh[l] & 3
            elif quarter == 1:
                lo, hi = qlh[l + 32] & 0xF, (qhh[l] >> 2) & 3
            elif quarter == 2:
                lo, hi = qlh[l] >> 4, (qhh[l] >> 4) & 3
            else:
                lo, hi = qlh[l + 32] >> 4, (qhh[l] >> 6) & 3
            q = (lo | (hi << 4)) - 32
            acc += d * int(sc[half * 8 + is_ + quarter * 2]) * q * float(x[i])
        ref[r] = acc
        W += blk
    cases["selftest_q6_k_32x256"] = (Q6_K, bytes(W), x[None, :], 32, 256, ref)
    # Q4_K 64x1024 sharding pattern (:2368-2404): reference output is the GEMV itself, here fp64
    x = np.array([np.float32(0.02) * np.float32((i % 9) - 4) for i in range(1024)], np.float32)
    W = b"".join(q4k_fill(r * 7 + sb) for r in range(64) for sb in range(4))
    ref = np.array([sum(q4k_ref_f64(W[(r * 4 + sb) * 144:(r * 4 + sb + 1) * 144], x[sb * 256:(sb + 1) * 256])
                        for sb in range(4)) for r in range(64)])
    cases["selftest_q4_k_64x1024"] = (Q4_K, W, x[None, :], 64, 1024, ref)
    return cases


def rand_cases(seed=1234):
    """Random well-formed blocks per type (normal fp16 scales), moderate shapes."""
    rng = np.random.default_rng(seed)
    specs = {Q8_0: (34, [0]), Q4_0: (18, [0]), Q4_K: (144, [0, 2]), Q6_K: (210, [208])}
    cases = {}
    for t, (bb, offs) in specs.items():
        bs = 32 if bb in (34, 18) else 256
        rows, cols = 16, 2048 + (512 if bs == 256 else 96)
        nblk = rows * cols // bs
        w = rng.integers(0, 256, size=(nblk, bb), dtype=np.uint8)
        for o in offs:
            hv = (np.abs(rng.standard_normal(nblk)) * 0.01).astype(np.float16).view(np.uint16)
            w[:, o] = hv & 0xFF
            w[:, o + 1] = hv >> 8
        X = rng.standard_normal((3, cols)).astype(np.float32)
        cases[f"rand_t{t}"] = (t, w.tobytes(), X, rows, cols)
    return cases


def main():
    ref = oracle.ref_lib()
    if ref is None:
        raise SystemExit("oracle/_ref is not built (make -C oracle ref); it is needed to write fixtures")
    dot = oracle.ref_lib().qvxr_dot_kernel().decode()
    for name, (t, data, n) in kat_dequant().items():
        w = np.frombuffer(data, np.uint8).copy()
        out = oracle.dequantize(t, w, n, use_ref=True)
        np.savez(os.path.join(HERE, f"kat_dequant_{name}.npz"), type=t, w=w, n=n, expected=out)
    for name, (t, data, X, rows, cols) in {**kat_qmatmul(), **rand_cases()}.items():
        w = np.frombuffer(data, np.uint8).copy()
        nvec = X.shape[0]
        out = oracle.qmatmul_n(w, t, X, nvec, rows, cols, use_ref=True)
        deq = oracle.dequantize(t, w, rows * cols, use_ref=True)
        prefix = "kat_qmatmul" if name in kat_qmatmul() else "rand"
        fname = f"{prefix}_{name}.npz" if prefix == "kat_qmatmul" else f"{name}.npz"
        np.savez(os.path.join(HERE, fname), type=t, w=w, X=X, rows=rows, cols=cols, expected=out,
                 dequant=deq, dot_kernel=dot)
    for name, (t, data, X, rows, cols, f64ref) in selftests().items():
        w = np.frombuffer(data, np.uint8).copy()
        out = oracle.qmatmul_n(w, t, X, 1, rows, cols, use_ref=True)
        np.savez(os.path.join(HERE, f"kat_{name}.npz"), type=t, w=w, X=X, rows=rows, cols=cols, expected=out,
                 f64ref=f64ref, dot_kernel=dot)
    print("fixtures written to", HERE)


if __name__ == "__main__":
    main()
