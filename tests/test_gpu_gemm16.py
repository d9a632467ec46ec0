"""The plain 16-bit matrix-core GEMM (qvx_gemm16, k_gemm16) and the prefill route built on it for the
weight types without a raw-block kernel: weight dequantised to 16 bits (qvx_dequantize16), then
k_gemm16.

qvx_gemm16 is checked on exactly representable operands: X and B are 16-bit values, so the exact
product is the fp64 sum of their fp32 values, and the only error left is fp32 accumulation (bar 1e-4
max-relative: a transposed operand, a wrong K chunk or a misplaced tile is off by O(1)).  The shapes
take both tile kernels (the 4-wave kernel on 256-token tiles, the 8-wave kernel on 128-token tiles),
ragged M and N, a K split, K not a multiple of 64 and unaligned operands (zero-padded copies).  The prefill route is held to the GEMM bar of the fp64 oracle at the BASELINE Q8_0 / Q4_0
shapes (a row slice), and its 16-bit weight to the oracle's dequantised value rounded once.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
import qorvix_amd as qvx
from conftest import max_rel

pytestmark = pytest.mark.gpu

EXACT_TOL = 1e-4
GEMM_TOL = 2e-2


def _bits16(a32, bf16):
    """fp32 -> 16-bit bits (round to nearest even) and the fp32 value those bits hold."""
    if bf16:
        u = a32.astype(np.float32).view(np.uint32).astype(np.uint64)
        b = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
        return b, (b.astype(np.uint32) << 16).view(np.float32)
    h = a32.astype(np.float16)
    return h.view(np.uint16), h.astype(np.float32)


def _gemm16(cuda, Xb, Bb, variant, x_off=0, b_off=0):
    """qvx_gemm16 on device copies placed x_off / b_off bytes into their buffers."""
    M, K = Xb.shape
    N = Bb.shape[0]
    bx = cuda.zeros(Xb.size * 2 + 64, dtype=cuda.uint8, device="cuda")
    bb = cuda.zeros(Bb.size * 2 + 64, dtype=cuda.uint8, device="cuda")
    bx[x_off:x_off + Xb.size * 2] = cuda.from_numpy(np.ascontiguousarray(Xb).view(np.uint8).reshape(-1)).cuda()
    bb[b_off:b_off + Bb.size * 2] = cuda.from_numpy(np.ascontiguousarray(Bb).view(np.uint8).reshape(-1)).cuda()
    out = cuda.full((M, N), float("nan"), dtype=cuda.float32, device="cuda")
    rc = qvx.lib().qvx_gemm16(out.data_ptr(), bx.data_ptr() + x_off, bb.data_ptr() + b_off, M, N, K, variant,
                              cuda.cuda.current_stream().cuda_stream)
    assert rc == qvx.OK, qvx.strerror(rc)
    cuda.cuda.synchronize()
    return out.cpu().numpy()


@pytest.mark.parametrize("variant", [qvx.GEMM_BF16, qvx.GEMM_F16])
@pytest.mark.parametrize("M,N,K,x_off,b_off", [
    (1900, 6500, 128, 0, 0),    # 4-wave kernel (26 x 8 = 208 tiles), ragged last tile in M and N
    (300, 520, 192, 0, 0),      # 8-wave kernel, ragged, three 64-element slices
    (2048, 11000, 128, 0, 0),   # two launches: 32 columns of 256-token tiles, 11 of 128-token tiles
    (128, 512, 2048, 0, 0),     # 2 tiles: four K splits of 8 slices, summed in split order
    (70, 100, 100, 0, 0),       # K not a multiple of 64: zero-padded copies of both operands
    (64, 256, 512, 2, 6),       # operands off 16-byte alignment: padded copies
    (1, 1, 64, 0, 0),           # one output
])
def test_gemm16_exact_operands(cuda, variant, M, N, K, x_off, b_off):
    bf16 = variant == qvx.GEMM_BF16
    rng = np.random.default_rng(M * 7 + N * 3 + K + variant)
    Xb, Xv = _bits16(rng.standard_normal((M, K)).astype(np.float32), bf16)
    Bb, Bv = _bits16(rng.standard_normal((N, K)).astype(np.float32), bf16)
    got = _gemm16(cuda, Xb, Bb, variant, x_off, b_off)
    ref = Xv.astype(np.float64) @ Bv.astype(np.float64).T
    assert np.isfinite(got).all()
    assert max_rel(got, ref) <= EXACT_TOL


def test_gemm16_deterministic(cuda):
    """The same call twice returns the same bits (a K split adds its partials in split order)."""
    rng = np.random.default_rng(11)
    Xb, _ = _bits16(rng.standard_normal((128, 4096)).astype(np.float32), True)
    Bb, _ = _bits16(rng.standard_normal((1024, 4096)).astype(np.float32), True)
    a = _gemm16(cuda, Xb, Bb, qvx.GEMM_BF16)
    b = _gemm16(cuda, Xb, Bb, qvx.GEMM_BF16)
    np.testing.assert_array_equal(a.view(np.uint32), b.view(np.uint32))


def test_gemm16_tile_kernels_agree_bitwise(cuda):
    """Without a K split both tile kernels add the K16 products of an output in the same order, so a
    256-token-tile call (M = 2048, N = 6656: 208 tiles) and 128-token-tile calls over row slices of
    the same operands (the slices run too few tiles for 256-token tiles) give the same bits."""
    rng = np.random.default_rng(12)
    Xb, _ = _bits16(rng.standard_normal((2048, 256)).astype(np.float32), False)
    Bb, _ = _bits16(rng.standard_normal((6656, 256)).astype(np.float32), False)
    whole = _gemm16(cuda, Xb, Bb, qvx.GEMM_F16)
    part = _gemm16(cuda, Xb, Bb[:1024], qvx.GEMM_F16)
    np.testing.assert_array_equal(whole[:, :1024].view(np.uint32), part.view(np.uint32))


@pytest.mark.parametrize("t", [qvx.Q8_0, qvx.Q4_0, qvx.Q4_K, qvx.Q6_K, qvx.Q5_0, qvx.Q5_K, qvx.F16])
@pytest.mark.parametrize("bf16", [True, False])
def test_dequantize16_bit_exact(cuda, t, bf16):
    """qvx_dequantize16 equals the oracle's dequantised fp32 value rounded once to bf16 / fp16."""
    rows, cols = 96, 512
    rng = np.random.default_rng(31 + t)
    from test_gpu_kernels import random_weight, dev
    w = random_weight(t, rows, cols, rng, scale=0.002)
    got = qvx.dequantize16_t(dev(cuda, w), t, rows * cols, bf16).cpu().numpy().view(np.uint16)
    want, _ = _bits16(oracle.dequantize(t, w, rows * cols).astype(np.float32), bf16)
    np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("t,rows,cols", [(qvx.Q8_0, 4096, 4096), (qvx.Q4_0, 11008, 4096), (qvx.Q4_0, 4096, 11008)])
@pytest.mark.parametrize("M", [512, 2048])
def test_prefill_via16_config_shapes(cuda, t, rows, cols, M):
    """BASELINE configs 1-2's Q8_0 and Q4_0 weights as prefill GEMMs (both 16-bit variants) against
    the fp64 oracle on a row slice, and the no-allocation entry point taking the same calls (its
    16-bit weight in panels of rows inside the scratch) within the same bar."""
    W = qvx.empty_weight(t, rows, cols)
    qvx.fill_synthetic_t(W, t, rows, cols, seed=300 + t + M, scale_mul=1e-3)
    X = cuda.empty((M, cols), dtype=cuda.float16, device="cuda")
    qvx.fill_normal_t(X, seed=301 + t + M, mul=0.5)
    cuda.cuda.synchronize()
    rb = qvx.row_bytes(t, cols)
    idx = np.union1d(np.arange(0, rows, 97), [rows - 1])
    Wd = oracle.dequantize(t, W.cpu().numpy().reshape(rows, rb)[idx].reshape(-1), len(idx) * cols)
    ref = X.cpu().numpy().astype(np.float64) @ Wd.reshape(len(idx), cols).astype(np.float64).T
    s = cuda.cuda.current_stream().cuda_stream
    for variant in (qvx.GEMM_BF16, qvx.GEMM_F16):
        out = qvx.qgemm_t(W, t, X, rows, cols, variant)
        cuda.cuda.synchronize()
        got = out.cpu().numpy()
        assert np.isfinite(got).all()
        assert max_rel(got[:, idx], ref) <= GEMM_TOL, variant
        out2 = cuda.full((M, rows), float("nan"), dtype=cuda.float32, device="cuda")
        rc = qvx.lib().qvx_qgemm_f16_noalloc(out2.data_ptr(), W.data_ptr(), t, X.data_ptr(), M, rows, cols, variant, s)
        assert rc == qvx.OK, qvx.strerror(rc)
        cuda.cuda.synchronize()
        got2 = out2.cpu().numpy()
        assert max_rel(got2[:, idx], ref) <= GEMM_TOL, variant


@pytest.mark.parametrize("bf16", [True, False])
def test_dequantize16_scale_edge_values(cuda, bf16):
    """16-bit dequantisation with fp16 scales at their extremes (subnormal, smallest normal, max,
    negative, signed zero) and extreme quants, against the oracle's value rounded once (fp16 overflow to
    Inf included).  The tensors end in a partial workgroup span, and Q8_0 / Q6_K in a span whose byte
    count is not a multiple of 16."""
    from test_gpu_kernels import dev
    specials = [0x0001, 0x03FF, 0x0400, 0x7BFF, 0x8001, 0xFBFF, 0x0000, 0x8000, 0x3C00]
    rng = np.random.default_rng(6)
    blocks = []
    for d in specials:
        for dm in specials:
            b = rng.integers(0, 256, 144, dtype=np.uint8)
            b[0], b[1], b[2], b[3] = d & 0xFF, d >> 8, dm & 0xFF, dm >> 8
            blocks.append(b)
    cases = [(qvx.Q4_K, np.concatenate(blocks), len(blocks) * 256)]
    for t, off, bb, qk in ((qvx.Q6_K, 208, 210, 256), (qvx.Q8_0, 0, 34, 32), (qvx.Q4_0, 0, 18, 32)):
        blocks = []
        for d in specials:
            for fill in (0x00, 0xFF, 0x80, 0x7F):
                b = np.full(bb, fill, np.uint8)
                b[off], b[off + 1] = d & 0xFF, d >> 8
                blocks.append(b)
        cases.append((t, np.concatenate(blocks), len(blocks) * qk))
    for t, w, n in cases:
        got = qvx.dequantize16_t(dev(cuda, w), t, n, bf16).cpu().numpy().view(np.uint16)
        with np.errstate(over="ignore"):
            want, _ = _bits16(oracle.dequantize(t, w, n).astype(np.float32), bf16)
        np.testing.assert_array_equal(got, want, err_msg=f"type {t}")


@pytest.mark.parametrize("t,rows,cols,M", [(qvx.Q8_0, 4096, 4096, 512), (qvx.Q4_0, 1024, 11008, 300),
                                           (qvx.Q5_K, 2048, 4096, 64), (qvx.Q8_0, 256, 4128, 40)])
def test_prefill_via16_bf16_is_its_composition(cuda, t, rows, cols, M):
    """The bf16 prefill route for these types rounds X to bf16 in the same launch that dequantises the
    weight (K a multiple of 64; the padded case 4128 takes its own prepass) and then runs the plain
    16-bit GEMM: its output equals, bit for bit, qvx_dequantize16's bf16 weight times X rounded to
    bf16 (to nearest even) through qvx_gemm16.  X carries +-Inf, NaN, a subnormal, fp16's largest
    value and -0 in its first row."""
    W = qvx.empty_weight(t, rows, cols)
    qvx.fill_synthetic_t(W, t, rows, cols, seed=400 + t + M, scale_mul=1e-3)
    X = cuda.empty((M, cols), dtype=cuda.float16, device="cuda")
    qvx.fill_normal_t(X, seed=401 + t + M, mul=0.5)
    X[0, :8] = cuda.tensor([float("inf"), -float("inf"), float("nan"), 6.0e-8, 65504.0, -0.0, 1 / 3, -2.5e-5],
                           dtype=cuda.float16, device="cuda")
    cuda.cuda.synchronize()
    got = qvx.qgemm_t(W, t, X, rows, cols, qvx.GEMM_BF16)
    B = qvx.dequantize16_t(W, t, rows * cols, True)
    xb, _ = _bits16(X.cpu().numpy().astype(np.float32), True)  # fp16 NaN -> 0x7FC0, as the kernel keeps it
    Xb = cuda.from_numpy(xb.view(np.int16)).cuda()
    ref = cuda.full((M, rows), float("nan"), dtype=cuda.float32, device="cuda")
    if cols % 64 == 0:
        rc = qvx.lib().qvx_gemm16(ref.data_ptr(), Xb.data_ptr(), B.data_ptr(), M, rows, cols, qvx.GEMM_BF16,
                                  cuda.cuda.current_stream().cuda_stream)
        assert rc == qvx.OK, qvx.strerror(rc)
        cuda.cuda.synchronize()
        np.testing.assert_array_equal(got.cpu().numpy(), ref.cpu().numpy())
    g = got.cpu().numpy()
    assert not np.isfinite(g[0]).any()  # the Inf / NaN activations reach every output of row 0
    assert np.isfinite(g[1:]).all()
