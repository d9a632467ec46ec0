"""CPU tests that pin the oracle (oracle/qvx_oracle.c) before it is trusted as the GPU checker.

Each check is chosen so that a plausible slip (wrong nibble order, dropped min term, wrong scale
index, sign of an int8, reassociated sum) fails at least one of them:
  * the reference's own known-answer tests, with their stated expected values;
  * fixtures holding the reference's own outputs (tests/golden, written from oracle/_ref);
  * exact rational arithmetic with one explicit round-to-nearest-even (closed form);
  * numpy's float16 decoder over all 65536 encodings;
  * brute-force Fraction sums for the fp64 oracle;
  * the reference built from its sources (oracle/_ref) on fresh random blocks, when present.
"""
from __future__ import annotations

from fractions import Fraction

import numpy as np
import pytest

import oracle
from conftest import golden, load_npz, max_rel

Q4_0, Q4_1, Q5_0, Q5_1, Q8_0, Q8_1, Q4_K, Q5_K, Q6_K, F16, BF16, F32 = 2, 3, 6, 7, 8, 9, 12, 13, 14, 1, 30, 0
BLOCK = {Q4_0: (32, 18), Q4_1: (32, 20), Q5_0: (32, 22), Q5_1: (32, 24), Q8_0: (32, 34), Q8_1: (32, 36),
         Q4_K: (256, 144), Q5_K: (256, 176), Q6_K: (256, 210), F16: (1, 2), BF16: (1, 2), F32: (1, 4)}
HALF_OFFS = {Q4_0: [0], Q4_1: [0, 2], Q5_0: [0], Q5_1: [0, 2], Q8_0: [0], Q8_1: [0, 2], Q4_K: [0, 2],
             Q5_K: [0, 2], Q6_K: [208]}


def f32bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


def random_blocks(t, nblk, rng, scale=0.01):
    bs, bb = BLOCK[t]
    w = rng.integers(0, 256, size=(nblk, bb), dtype=np.uint8)
    for o in HALF_OFFS.get(t, []):
        hv = (np.abs(rng.standard_normal(nblk)) * scale + 1e-4).astype(np.float16).view(np.uint16)
        w[:, o] = hv & 0xFF
        w[:, o + 1] = hv >> 8
    return w.reshape(-1)


# ---- exact closed form ---------------------------------------------------------------------------

NEG_ZERO = "-0"


def rn_f32(v: Fraction) -> np.float32:
    """Round an exact rational to float32, ties to even (normal range)."""
    if isinstance(v, str):
        return np.float32(-0.0)
    if v == 0:
        return np.float32(0.0)
    sign = -1 if v < 0 else 1
    v = abs(v)
    e = v.numerator.bit_length() - v.denominator.bit_length()
    # scale so that the integer part has exactly 24 bits
    shift = 23 - e
    while True:
        scaled = v * (Fraction(2) ** shift)
        q = scaled.numerator // scaled.denominator
        if q >= (1 << 24):
            shift -= 1
        elif q < (1 << 23):
            shift += 1
        else:
            break
    r = scaled - q
    if r > Fraction(1, 2) or (r == Fraction(1, 2) and q % 2 == 1):
        q += 1
    return np.float32(sign * float(Fraction(q) / (Fraction(2) ** shift)))


def hfrac(lo, hi) -> Fraction:
    return Fraction(float(np.array([lo | (hi << 8)], np.uint16).view(np.float16)[0]))


def exact_dequant(t, blk) -> list:
    """Dequantised values of one block as exact rationals (public GGUF definitions)."""
    b = [int(v) for v in blk]
    out = []
    if t == Q8_0:
        d = hfrac(b[0], b[1])
        out = [d * (b[2 + i] - 256 if b[2 + i] > 127 else b[2 + i]) for i in range(32)]
    elif t == Q4_0:
        d = hfrac(b[0], b[1])
        out = [d * ((b[2 + i] & 15) - 8) for i in range(16)] + [d * ((b[2 + i] >> 4) - 8) for i in range(16)]
    elif t == Q4_K:
        d, dmin = hfrac(b[0], b[1]), hfrac(b[2], b[3])
        s = b[4:16]
        for c in range(4):
            for half in range(2):
                j = 2 * c + half
                if j < 4:
                    sc, m = s[j] & 63, s[j + 4] & 63
                else:
                    sc, m = (s[j + 4] & 15) | ((s[j - 4] >> 6) << 4), (s[j + 4] >> 4) | ((s[j] >> 6) << 4)
                for l in range(32):
                    q = b[16 + 32 * c + l]
                    n = (q >> 4) if half else (q & 15)
                    out.append(d * sc * n - dmin * m)
    elif t == Q6_K:
        d = hfrac(b[208], b[209])
        vals = [None] * 256
        for h in range(2):
            for l in range(32):
                for quarter in range(4):
                    lo = b[64 * h + l + (32 if quarter & 1 else 0)]
                    nib = (lo >> 4) if quarter & 2 else (lo & 15)
                    q = nib | (((b[128 + 32 * h + l] >> (2 * quarter)) & 3) << 4)
                    sc = b[192 + 8 * h + l // 16 + 2 * quarter]
                    sc = sc - 256 if sc > 127 else sc
                    # IEEE products of zero carry the xor of the factor signs (integer 0 is +0.0)
                    v = d * sc * (q - 32)
                    neg = (d < 0) ^ (sc < 0) ^ (q - 32 < 0)
                    vals[128 * h + 32 * quarter + l] = NEG_ZERO if (v == 0 and neg) else v
        out = vals
    return out


@pytest.mark.parametrize("t", [Q8_0, Q4_0, Q4_K, Q6_K])
def test_dequant_equals_rounded_exact_value(t):
    rng = np.random.default_rng(100 + t)
    bs, bb = BLOCK[t]
    nblk = 24
    w = random_blocks(t, nblk, rng)
    got = oracle.dequantize(t, w, nblk * bs)
    want = np.array([rn_f32(v) for k in range(nblk) for v in exact_dequant(t, w[k * bb:(k + 1) * bb])], np.float32)
    np.testing.assert_array_equal(f32bits(got), f32bits(want))


def test_rn_f32_helper_rounds_ties_to_even():
    # 1 + 2^-24 is a tie between 1 and 1 + 2^-23: even mantissa (1.0) wins; 1 + 3*2^-24 rounds up.
    assert rn_f32(Fraction(1) + Fraction(1, 2 ** 24)) == np.float32(1.0)
    assert rn_f32(Fraction(1) + Fraction(3, 2 ** 24)) == np.float32(1.0 + 2 ** -22)
    assert rn_f32(Fraction(-5, 3)) == np.float32(-5 / 3)


def test_fp16_decode_all_encodings():
    # through the F16 dequantiser, so values (signalling-NaN payloads included) stay in memory
    # and are never converted by ctypes' float -> double return path
    bits = np.arange(65536, dtype=np.uint16)
    want = f32bits(bits.view(np.float16).astype(np.float32))
    got = oracle.dequantize(F16, bits.view(np.uint8), 65536)
    np.testing.assert_array_equal(f32bits(got), want)
    lib = oracle.lib()  # the scalar entry point agrees on every non-NaN encoding
    finite = bits[(bits & 0x7C00) != 0x7C00]
    np.testing.assert_array_equal(np.array([lib.qvxo_fp16_to_float(int(h)) for h in finite], np.float32),
                                  finite.view(np.float16).astype(np.float32))


def test_bf16_decode():
    lib = oracle.lib()
    for b in [0x3F80, 0x4040, 0x0000, 0x8000, 0x7F80, 0x0001]:
        assert f32bits(np.float32(lib.qvxo_bf16_to_float(b))) == np.uint32(b << 16)


def test_type_traits_table():
    assert oracle.traits(2) == (32, 18) and oracle.traits(8) == (32, 34)
    assert oracle.traits(12) == (256, 144) and oracle.traits(14) == (256, 210)
    assert oracle.traits(4) is None and oracle.traits(31) is None
    lib = oracle.lib()
    assert lib.qvxo_can_dequantize(Q4_K) and lib.qvxo_can_dequantize(F16)
    assert not lib.qvxo_can_dequantize(10) and not lib.qvxo_can_dequantize(16)
    assert not lib.qvxo_supports(10)  # Q2_K: qmatmul_test.cpp:96


# ---- the reference's known-answer tests ----------------------------------------------------------

KAT_EXPECT = {
    # dequant_test.cpp stated values
    "q8_0_pos": lambda: np.array([0.5 * i for i in range(32)], np.float32),
    "q8_0_neg": lambda: np.array([-i for i in range(32)], np.float32),
    "q4_0_split": lambda: np.array([-8.0] * 16 + [0.0] * 16, np.float32),
    "q4_1": lambda: np.array([2.5] * 16 + [6.5] * 16, np.float32),
    "q5_0_qh0": lambda: np.full(32, -16.0, np.float32),
    "q6_k_uniform": lambda: np.full(256, -32.0, np.float32),
    "q4_k_uniform": lambda: np.zeros(256, np.float32),
    "f16_known": lambda: np.array([1.0, 0.5, 0.0, -2.0], np.float32),
    "bf16_known": lambda: np.array([1.0, 3.0], np.float32),
}


@pytest.mark.parametrize("path", golden("kat_dequant_*.npz"))
def test_kat_dequant(path):
    d = load_npz(path)
    name = path.split("kat_dequant_")[1][:-4]
    got = oracle.dequantize(int(d["type"]), d["w"], int(d["n"]))
    np.testing.assert_array_equal(f32bits(got), f32bits(d["expected"]))  # the reference's own output
    if name in KAT_EXPECT:
        np.testing.assert_array_equal(got, KAT_EXPECT[name]())
    if name == "q5_0_qh1":
        assert got[0] == 0.0 and got[1] == -16.0
    if name == "q6_k_one":
        assert got[0] == -17.0 and np.all(got[1:] == -32.0)
    if name == "q4_k_one":
        assert got[0] == 5.0 and np.all(got[1:] == 0.0)


@pytest.mark.parametrize("path", golden("kat_qmatmul_*.npz"))
def test_kat_qmatmul(path):
    d = load_npz(path)
    t, rows, cols, X = int(d["type"]), int(d["rows"]), int(d["cols"]), d["X"]
    got = oracle.qmatmul_n(d["w"], t, X, X.shape[0], rows, cols)
    # the reference's own test oracle: dequantize everything, then an F32 GEMV (qmatmul_test.cpp:30-37)
    deq = oracle.dequantize(t, d["w"], rows * cols).reshape(rows, cols).astype(np.float64)
    tol = 1e-2 if t == Q4_K else 1e-3
    np.testing.assert_allclose(got, X.astype(np.float64) @ deq.T, atol=tol, rtol=0)
    if str(d["dot_kernel"]) == oracle.lib().qvxo_dot_kernel().decode():
        np.testing.assert_array_equal(f32bits(got), f32bits(d["expected"]))
    else:
        np.testing.assert_allclose(got, d["expected"], rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("path", golden("kat_selftest_*.npz"))
def test_kat_cuda_selftest_patterns(path):
    d = load_npz(path)
    t, rows, cols, X = int(d["type"]), int(d["rows"]), int(d["cols"]), d["X"]
    got = oracle.qmatmul(d["w"], t, X[0], rows, cols)
    assert max_rel(got, d["f64ref"]) < 1e-3  # the self-tests' own gate (cuda_backend.cu:766-774)
    f64 = oracle.matmul_f64(d["w"], t, X, 1, rows, cols)[0]
    assert max_rel(f64, d["f64ref"]) < 1e-12
    if str(d["dot_kernel"]) == oracle.lib().qvxo_dot_kernel().decode():
        np.testing.assert_array_equal(f32bits(got), f32bits(d["expected"][0]))


@pytest.mark.parametrize("path", golden("rand_*.npz"))
def test_random_fixtures(path):
    d = load_npz(path)
    t, rows, cols, X = int(d["type"]), int(d["rows"]), int(d["cols"]), d["X"]
    np.testing.assert_array_equal(f32bits(oracle.dequantize(t, d["w"], rows * cols)), f32bits(d["dequant"]))
    got = oracle.qmatmul_n(d["w"], t, X, X.shape[0], rows, cols)
    if str(d["dot_kernel"]) == oracle.lib().qvxo_dot_kernel().decode():
        np.testing.assert_array_equal(f32bits(got), f32bits(d["expected"]))
    assert max_rel(got, oracle.matmul_f64(d["w"], t, X, X.shape[0], rows, cols)) < 1e-5


# ---- operator behaviour --------------------------------------------------------------------------

def test_qmatmul_n_bit_identical_to_qmatmul():
    rng = np.random.default_rng(7)
    for t, rows, cols, nvec in [(Q8_0, 12, 64, 5), (Q4_K, 9, 512, 70), (Q6_K, 5, 768, 3), (Q4_0, 33, 96, 17)]:
        bs, bb = BLOCK[t]
        w = random_blocks(t, rows * cols // bs, rng)
        X = rng.standard_normal((nvec, cols)).astype(np.float32)
        batched = oracle.qmatmul_n(w, t, X, nvec, rows, cols)
        for v in range(nvec):
            np.testing.assert_array_equal(f32bits(batched[v]), f32bits(oracle.qmatmul(w, t, X[v], rows, cols)))


def test_rejections_match_reference():
    w = np.zeros(34, np.uint8)
    x = np.ones(30, np.float32)
    assert oracle.qmatmul(w, Q8_0, x, 1, 30) is None  # cols % 32 (qmatmul_test.cpp:89-97)
    assert oracle.qmatmul_n(w, Q8_0, x, 0, 1, 32) is None  # nVec <= 0 (qmatmul.cpp:66)
    assert oracle.qmatmul(w, 10, x, 1, 256) is None  # Q2_K unsupported
    assert oracle.dequant_row(w, 4, 32, 0) is None  # unknown type id


def test_dequant_row_selects_row():
    # qmatmul_test.cpp:79-87: rows of Q8_0 blocks d=1, qs = 10r + i
    w = bytearray()
    for r in range(4):
        w += bytes([0x00, 0x3C]) + bytes((10 * r + i) & 0xFF for i in range(32))
    row = oracle.dequant_row(np.frombuffer(bytes(w), np.uint8), Q8_0, 32, 2)
    np.testing.assert_array_equal(row, np.arange(20, 52, dtype=np.float32))


def test_matmul_f64_brute_force():
    rng = np.random.default_rng(3)
    for t in (Q8_0, Q4_0, Q4_K, Q6_K):
        bs, bb = BLOCK[t]
        rows, cols, nvec = 3, bs * 2, 2
        w = random_blocks(t, rows * cols // bs, rng)
        X = rng.standard_normal((nvec, cols)).astype(np.float32)
        got = oracle.matmul_f64(w, t, X, nvec, rows, cols)
        for r in range(rows):
            vals = [v for b in range(cols // bs) for v in exact_dequant(t, w[(r * (cols // bs) + b) * bb:][:bb])]
            for v in range(nvec):
                exact = sum(Fraction(float(rn_f32(a))) * Fraction(float(xk)) for a, xk in zip(vals, X[v]))
                assert abs(got[v, r] - float(exact)) <= 1e-12 * max(1.0, abs(float(exact)))


def test_quantize_q8_act_properties():
    rng = np.random.default_rng(11)
    X = (rng.standard_normal((4, 256)) * 0.5).astype(np.float16).astype(np.float32)
    X[1, 32:64] = 0.0  # an all-zero block
    q, s, qs = oracle.quantize_q8_act(X)
    blocks = X.reshape(4, 8, 32)
    qb = q.reshape(4, 8, 32).astype(np.int32)
    amax = np.abs(blocks).max(axis=2)
    np.testing.assert_array_equal(s, (amax / np.float32(127)).astype(np.float32))
    assert np.all(np.abs(qb) <= 127)
    np.testing.assert_array_equal(qs, qb.sum(axis=2))
    assert s[1, 1] == 0 and np.all(qb[1, 1] == 0)
    # the block maximum maps to +-127 and reconstruction error is within half a step
    for m in range(4):
        for j in range(8):
            if amax[m, j] > 0:
                k = int(np.argmax(np.abs(blocks[m, j])))
                assert abs(qb[m, j, k]) == 127
                assert np.all(np.abs(qb[m, j] * s[m, j] - blocks[m, j]) <= 0.5 * s[m, j] * (1 + 1e-5))
    # round half away from zero: 0.5 -> 1 and -0.5 -> -1 in units of the step
    Xh = np.zeros((1, 32), np.float32)
    Xh[0, 0], Xh[0, 1], Xh[0, 2] = 127.0, 0.5, -0.5
    qh, _, _ = oracle.quantize_q8_act(Xh)
    assert qh[0, 0] == 127 and qh[0, 1] == 1 and qh[0, 2] == -1


# ---- against the reference built from its own sources ----------------------------------------------

needs_ref = pytest.mark.skipif(oracle.ref_lib() is None, reason="oracle/_ref not built (reference tree absent)")


@needs_ref
@pytest.mark.parametrize("t", [Q8_0, Q8_1, Q4_0, Q4_1, Q5_0, Q5_1, Q4_K, Q5_K, Q6_K, F16, BF16, F32])
def test_oracle_matches_reference_build(t):
    rng = np.random.default_rng(500 + t)
    bs, bb = BLOCK[t]
    rows, cols = 37, (2048 + 512) if bs != 1 else 300
    if bs == 1:
        if t == F32:
            w = rng.standard_normal(rows * cols).astype(np.float32).view(np.uint8)
        else:
            w = (rng.standard_normal(rows * cols) if t == F16 else rng.standard_normal(rows * cols)).astype(
                np.float16).view(np.uint8) if t == F16 else (
                rng.standard_normal(rows * cols).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16).view(np.uint8)
    else:
        w = random_blocks(t, rows * cols // bs, rng)
    n = rows * cols
    np.testing.assert_array_equal(f32bits(oracle.dequantize(t, w, n)), f32bits(oracle.dequantize(t, w, n, use_ref=True)))
    X = rng.standard_normal((3, cols)).astype(np.float32)
    a = oracle.qmatmul(w, t, X[0], rows, cols)
    b = oracle.qmatmul(w, t, X[0], rows, cols, use_ref=True)
    np.testing.assert_array_equal(f32bits(a), f32bits(b))
    np.testing.assert_array_equal(f32bits(oracle.qmatmul_n(w, t, X, 3, rows, cols)),
                                  f32bits(oracle.qmatmul_n(w, t, X, 3, rows, cols, use_ref=True)))
    np.testing.assert_array_equal(f32bits(oracle.dequant_row(w, t, cols, 5)),
                                  f32bits(oracle.dequant_row(w, t, cols, 5, use_ref=True)))


@needs_ref
def test_oracle_rejections_match_reference_build():
    ref, lib = oracle.ref_lib(), oracle.lib()
    for t in range(0, 40):
        assert bool(ref.qvxr_supports(t)) == bool(lib.qvxo_supports(t)), t
        assert bool(ref.qvxr_can_dequantize(t)) == bool(lib.qvxo_can_dequantize(t)), t
    w = np.zeros(4096, np.uint8)
    x = np.ones(512, np.float32)
    for t, cols in [(Q8_0, 30), (Q4_K, 300), (2, 40), (10, 256), (16, 256)]:
        assert (oracle.qmatmul(w, t, x, 1, cols) is None) == (oracle.qmatmul(w, t, x, 1, cols, use_ref=True) is None)


# ---- rmsnorm / swiglu (runtime/src/ops.cpp:8-13, 96-100) -----------------------------------------

@needs_ref
@pytest.mark.parametrize("n,eps", [(4096, 1e-5), (512, 1e-6), (7, 0.0), (14336, 1e-5)])
def test_rmsnorm_matches_reference_build(n, eps):
    rng = np.random.default_rng(n)
    x = (rng.standard_normal((3, n)) * rng.uniform(0.01, 30.0)).astype(np.float32)
    w = rng.standard_normal(n).astype(np.float32)
    a, b = oracle.rmsnorm(x, w, eps), oracle.rmsnorm(x, w, eps, use_ref=True)
    np.testing.assert_array_equal(a.view(np.uint32), b.view(np.uint32))


@needs_ref
def test_swiglu_matches_reference_build():
    rng = np.random.default_rng(5)
    g = np.concatenate([rng.standard_normal(4000) * 6, [0.0, -0.0, 88.0, -88.0, 1e-30, -200.0, 200.0]]).astype(np.float32)
    u = rng.standard_normal(g.size).astype(np.float32)
    a, b = oracle.swiglu(g, u), oracle.swiglu(g, u, use_ref=True)
    np.testing.assert_array_equal(a.view(np.uint32), b.view(np.uint32))


def test_rmsnorm_invariants():
    """What the definition fixes: with unit weights and eps = 0 the output's mean square is 1 and the
    output does not change when x is scaled by a power of two; a constant vector maps to +-1; the
    weight multiplies elementwise; eps bounds the scale of a zero vector."""
    rng = np.random.default_rng(11)
    n = 4096
    x = rng.standard_normal((2, n)).astype(np.float32)
    ones = np.ones(n, np.float32)
    y = oracle.rmsnorm(x, ones, 0.0).astype(np.float64)
    assert abs(float(np.mean(y * y, axis=1).max()) - 1.0) < 1e-5
    np.testing.assert_array_equal(oracle.rmsnorm(x * np.float32(8.0), ones, 0.0), oracle.rmsnorm(x, ones, 0.0))
    c = np.full((1, 100), -3.5, np.float32)
    np.testing.assert_allclose(oracle.rmsnorm(c, np.ones(100, np.float32), 0.0), -1.0, rtol=1e-6)
    w = rng.standard_normal(n).astype(np.float32)
    np.testing.assert_allclose(oracle.rmsnorm(x, w, 1e-5), oracle.rmsnorm(x, ones, 1e-5) * w, rtol=1e-6)
    z = np.zeros((1, 64), np.float32)
    np.testing.assert_array_equal(oracle.rmsnorm(z, np.ones(64, np.float32), 1e-5), z)


def test_swiglu_invariants():
    """silu(0) = 0; silu(z) -> z for large z and -> 0 for very negative z; silu(z) - silu(-z) = z;
    swiglu is linear in up."""
    z = np.array([0.0, 30.0, -30.0, 2.0, -2.0, 0.5], np.float32)
    one = np.ones_like(z)
    s = oracle.swiglu(z, one).astype(np.float64)
    assert s[0] == 0.0
    assert abs(s[1] - 30.0) < 1e-6 and abs(s[2]) < 1e-10
    np.testing.assert_allclose(s[3] - s[4], 2.0, rtol=1e-6)
    np.testing.assert_allclose(s[3], 2.0 / (1.0 + np.exp(-2.0)), rtol=1e-6)
    u = np.linspace(-3, 3, z.size).astype(np.float32)
    np.testing.assert_allclose(oracle.swiglu(z, 2 * u), 2 * oracle.swiglu(z, u), rtol=1e-6)
