"""GPU parity tests: the gfx950 kernels through the C ABI against the oracle (oracle/qvx_oracle.c)
and the reference's own outputs (tests/golden).

Bars: dequantisation bit-exact; GEMV max|y-ref|/max|ref| <= 1e-3 against the
fp64 sum of exact dequant values (fp32 accumulation); GEMM <= 2e-2 (16-bit MFMA path).
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
import qorvix_amd as qvx
from conftest import golden, load_npz, max_rel

pytestmark = pytest.mark.gpu

GEMV_TOL = 1e-3
GEMM_TOL = 2e-2
BLOCK = {qvx.Q4_0: (32, 18), qvx.Q4_1: (32, 20), qvx.Q5_0: (32, 22), qvx.Q5_1: (32, 24), qvx.Q8_0: (32, 34),
         qvx.Q8_1: (32, 36), qvx.Q4_K: (256, 144), qvx.Q5_K: (256, 176), qvx.Q6_K: (256, 210),
         qvx.F16: (1, 2), qvx.BF16: (1, 2), qvx.F32: (1, 4)}
HALF_OFFS = {qvx.Q4_0: [0], qvx.Q4_1: [0, 2], qvx.Q5_0: [0], qvx.Q5_1: [0, 2], qvx.Q8_0: [0], qvx.Q8_1: [0, 2],
             qvx.Q4_K: [0, 2], qvx.Q5_K: [0, 2], qvx.Q6_K: [208]}
GEMV_TYPES = [qvx.Q8_0, qvx.Q4_0, qvx.Q5_0, qvx.Q4_K, qvx.Q5_K, qvx.Q6_K]


def f32bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


def random_weight(t, rows, cols, rng, scale=0.01):
    bs, bb = BLOCK[t]
    nblk = rows * cols // bs
    if bs == 1:
        if t == qvx.F32:
            return rng.standard_normal(rows * cols).astype(np.float32).view(np.uint8)
        if t == qvx.F16:
            return rng.standard_normal(rows * cols).astype(np.float16).view(np.uint8)
        return (rng.standard_normal(rows * cols).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16).view(np.uint8)
    w = rng.integers(0, 256, size=(nblk, bb), dtype=np.uint8)
    for o in HALF_OFFS[t]:
        hv = (np.abs(rng.standard_normal(nblk)) * scale + 1e-4).astype(np.float16).view(np.uint16)
        w[:, o] = hv & 0xFF
        w[:, o + 1] = hv >> 8
    return w.reshape(-1)


def dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def run_gemv(torch, w_np, t, X_np, rows, cols, offset=0):
    """qvx_qmatmul_n on device copies; offset shifts the weight base (alignment cases)."""
    nvec = X_np.shape[0]
    buf = torch.zeros(w_np.size + 64, dtype=torch.uint8, device="cuda")
    buf[offset:offset + w_np.size] = dev(torch, w_np)
    X = dev(torch, X_np.astype(np.float32))
    out = torch.full((nvec, rows), float("nan"), dtype=torch.float32, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    if nvec == 1:
        rc = qvx.qmatmul(out.data_ptr(), buf.data_ptr() + offset, t, X.data_ptr(), rows, cols, stream)
    else:
        rc = qvx.qmatmul_n(out.data_ptr(), buf.data_ptr() + offset, t, X.data_ptr(), nvec, rows, cols, stream)
    assert rc == qvx.OK, qvx.strerror(rc)
    torch.cuda.synchronize()
    return out.cpu().numpy()


# ---- dequantisation: bit-exact --------------------------------------------------------------------

@pytest.mark.parametrize("t", sorted(BLOCK))
def test_dequant_bit_exact(cuda, t):
    rng = np.random.default_rng(40 + t)
    bs, bb = BLOCK[t]
    rows, cols = 33, (1024 if bs > 1 else 1000)
    w = random_weight(t, rows, cols, rng)
    n = rows * cols
    got = qvx.dequantize_t(dev(cuda, w), t, n)
    cuda.cuda.synchronize()
    want = oracle.dequantize(t, w, n)
    np.testing.assert_array_equal(f32bits(got.cpu().numpy()), f32bits(want))


@pytest.mark.parametrize("t", [qvx.Q8_0, qvx.Q4_0, qvx.Q4_K, qvx.Q5_K, qvx.Q6_K, qvx.Q5_1])
def test_dequant_unaligned_buffers(cuda, t):
    """Blocks 2 bytes off 4-byte alignment and an output 4 bytes off 16-byte alignment take the
    unstaged kernel; aligned ones the LDS-staged kernel, whose last workgroup is partial here.  Both
    are bit-exact, and the unstaged one writes nothing outside its output."""
    rng = np.random.default_rng(60 + t)
    rows, cols = 9, 768
    w = random_weight(t, rows, cols, rng)
    n = rows * cols
    want = f32bits(oracle.dequantize(t, w, n))
    raw = cuda.zeros(w.size + 16, dtype=cuda.uint8, device="cuda")
    raw[2:2 + w.size].copy_(cuda.from_numpy(w))
    buf = cuda.full((n + 8,), 7.0, dtype=cuda.float32, device="cuda")
    st = cuda.cuda.current_stream().cuda_stream
    assert qvx.lib().qvx_dequantize(t, raw.data_ptr() + 2, buf.data_ptr() + 4, n, st) == qvx.OK
    cuda.cuda.synchronize()
    got = buf.cpu().numpy()
    np.testing.assert_array_equal(f32bits(got[1:1 + n]), want)
    assert got[0] == 7.0 and np.all(got[1 + n:] == 7.0)
    aligned = qvx.dequantize_t(dev(cuda, w), t, n)
    cuda.cuda.synchronize()
    np.testing.assert_array_equal(f32bits(aligned.cpu().numpy()), want)


@pytest.mark.parametrize("t", [qvx.Q8_0, qvx.Q4_K, qvx.Q6_K])
def test_dequant_floors_to_whole_blocks(cuda, t):
    """n not a whole number of blocks: the reference converts n / blockSize blocks and leaves the rest
    of dst as it was (dequant.cpp:38-210); so does qvx_dequantize, on both host and device forms."""
    rng = np.random.default_rng(70 + t)
    bs, _ = BLOCK[t]
    w = random_weight(t, 3, 2 * bs, rng)
    n = 5 * bs + bs // 2 + 1  # five whole blocks and part of a sixth
    want = oracle.dequantize(t, w, 6 * bs)
    buf = cuda.full((6 * bs,), 7.0, dtype=cuda.float32, device="cuda")
    assert qvx.dequantize(t, dev(cuda, w).data_ptr(), buf.data_ptr(), n,
                          cuda.cuda.current_stream().cuda_stream) == qvx.OK
    cuda.cuda.synchronize()
    got = buf.cpu().numpy()
    np.testing.assert_array_equal(f32bits(got[:5 * bs]), f32bits(want[:5 * bs]))
    assert np.all(got[5 * bs:] == 7.0)
    host = np.full(6 * bs, 7.0, np.float32)
    assert qvx.lib().qvx_dequantize_host(t, w.ctypes.data, host.ctypes.data, n) == qvx.OK
    np.testing.assert_array_equal(f32bits(host), f32bits(got))


def test_dequant_fp16_scale_edge_values(cuda):
    """Scales at fp16 extremes: subnormal, smallest normal, max, negative, zero; quants at 0/15/63."""
    t = qvx.Q4_K
    specials = [0x0001, 0x03FF, 0x0400, 0x7BFF, 0x8001, 0xFBFF, 0x0000, 0x8000, 0x3C00]
    rng = np.random.default_rng(5)
    blocks = []
    for d in specials:
        for dm in specials:
            b = rng.integers(0, 256, 144, dtype=np.uint8)
            b[0], b[1], b[2], b[3] = d & 0xFF, d >> 8, dm & 0xFF, dm >> 8
            blocks.append(b)
    w = np.concatenate(blocks)
    n = len(blocks) * 256
    got = qvx.dequantize_t(dev(cuda, w), t, n).cpu().numpy()
    np.testing.assert_array_equal(f32bits(got), f32bits(oracle.dequantize(t, w, n)))
    # Q6_K / Q8_0 with the same scale set and extreme quants
    for t, off, bb in ((qvx.Q6_K, 208, 210), (qvx.Q8_0, 0, 34), (qvx.Q4_0, 0, 18)):
        blocks = []
        for d in specials:
            for fill in (0x00, 0xFF, 0x80, 0x7F):
                b = np.full(bb, fill, np.uint8)
                b[off], b[off + 1] = d & 0xFF, d >> 8
                blocks.append(b)
        w = np.concatenate(blocks)
        n = len(blocks) * BLOCK[t][0]
        got = qvx.dequantize_t(dev(cuda, w), t, n).cpu().numpy()
        np.testing.assert_array_equal(f32bits(got), f32bits(oracle.dequantize(t, w, n)))


@pytest.mark.parametrize("path", golden("kat_dequant_*.npz"))
def test_golden_dequant(cuda, path):
    d = load_npz(path)
    t, n = int(d["type"]), int(d["n"])
    got = qvx.dequantize_t(dev(cuda, d["w"]), t, n).cpu().numpy()
    np.testing.assert_array_equal(f32bits(got), f32bits(d["expected"]))


def test_dequant_row(cuda):
    rng = np.random.default_rng(9)
    for t in GEMV_TYPES:
        rows, cols = 7, 512
        w = random_weight(t, rows, cols, rng)
        W = dev(cuda, w)
        for row in (0, 3, 6):
            out = cuda.zeros(cols, dtype=cuda.float32, device="cuda")
            rc = qvx.dequant_row(W.data_ptr(), t, cols, row, out.data_ptr(), cuda.cuda.current_stream().cuda_stream)
            assert rc == qvx.OK
            cuda.cuda.synchronize()
            np.testing.assert_array_equal(f32bits(out.cpu().numpy()), f32bits(oracle.dequant_row(w, t, cols, row)))


# ---- GEMV ----------------------------------------------------------------------------------------

@pytest.mark.parametrize("path", golden("kat_qmatmul_*.npz") + golden("kat_selftest_*.npz") + golden("rand_*.npz"))
def test_golden_gemv(cuda, path):
    d = load_npz(path)
    t, rows, cols, X = int(d["type"]), int(d["rows"]), int(d["cols"]), d["X"]
    got = run_gemv(cuda, d["w"], t, X, rows, cols)
    ref = oracle.matmul_f64(d["w"], t, X, X.shape[0], rows, cols)
    assert max_rel(got, ref) <= GEMV_TOL
    assert max_rel(got, d["expected"].reshape(got.shape)) <= GEMV_TOL  # the reference's own output
    if "f64ref" in d:
        assert max_rel(got[0], d["f64ref"]) <= GEMV_TOL


SHAPES = [
    (1, 256), (3, 512), (17, 2048), (64, 2304), (100, 4096), (257, 4352),  # ragged rows, partial panels
    (4096, 4096), (1024, 14336),
]


@pytest.mark.parametrize("t", GEMV_TYPES)
@pytest.mark.parametrize("rows,cols", SHAPES)
def test_gemv_m1_parity(cuda, t, rows, cols):
    bs, _ = BLOCK[t]
    if cols % bs:
        pytest.skip("shape not a whole number of blocks")
    rng = np.random.default_rng(rows * 7 + cols + t)
    w = random_weight(t, rows, cols, rng)
    x = rng.standard_normal((1, cols)).astype(np.float32)
    got = run_gemv(cuda, w, t, x, rows, cols)
    ref = oracle.matmul_f64(w, t, x, 1, rows, cols)
    assert max_rel(got, ref) <= GEMV_TOL


@pytest.mark.parametrize("t", GEMV_TYPES)
@pytest.mark.parametrize("nvec", [2, 3, 4, 7, 8, 16, 17, 33])
def test_gemv_batched_parity_and_bit_identity(cuda, t, nvec):
    rng = np.random.default_rng(100 + nvec + t)
    rows, cols = 300, 4096
    w = random_weight(t, rows, cols, rng)
    X = rng.standard_normal((nvec, cols)).astype(np.float32)
    got = run_gemv(cuda, w, t, X, rows, cols)
    assert max_rel(got, oracle.matmul_f64(w, t, X, nvec, rows, cols)) <= GEMV_TOL
    # each vector bit-identical to the single-vector GEMV (qmatmul.hpp:31-32)
    for v in range(nvec):
        single = run_gemv(cuda, w, t, X[v:v + 1], rows, cols)
        np.testing.assert_array_equal(f32bits(got[v]), f32bits(single[0]))


@pytest.mark.parametrize("rows,cols,nvec", [(14336, 4096, 8), (1024, 4096, 5), (17, 2048, 3), (64, 2304, 8),
                                             (4096, 4096, 16)])
def test_gemv_q4k_batched_form_bit_identical(cuda, rows, cols, nvec):
    """The batched matrix-core form (2..8 vectors a launch) across the launch geometries (TQ x KQ
    splits, ragged rows): within tolerance of the oracle and bit-identical to one-vector calls."""
    t = qvx.Q4_K
    rng = np.random.default_rng(rows + 3 * cols + nvec)
    w = random_weight(t, rows, cols, rng)
    X = rng.standard_normal((nvec, cols)).astype(np.float32)
    got = run_gemv(cuda, w, t, X, rows, cols)
    assert max_rel(got, oracle.matmul_f64(w, t, X, nvec, rows, cols)) <= GEMV_TOL
    for v in range(nvec):
        single = run_gemv(cuda, w, t, X[v:v + 1], rows, cols)
        np.testing.assert_array_equal(f32bits(got[v]), f32bits(single[0]))


@pytest.mark.parametrize("rows,cols,nvec", [(300, 2048, 12), (17, 2048, 16), (1000, 14336, 13), (4099, 4096, 16),
                                             (64, 6144, 12), (8200, 4096, 5), (4096, 2048, 8), (257, 4096, 20),
                                             (4096, 14336, 3), (2048, 8192, 4), (33, 14336, 8), (5000, 2048, 6),
                                             (14336, 4096, 9), (700, 4096, 24), (300, 4096, 3), (8200, 2048, 4)])
def test_gemv_q6k_batched_form_bit_identical(cuda, rows, cols, nvec):
    """The batched matrix-core Q6_K form (8 or 16 vectors a launch, K a multiple of 2048, the K range
    split over workgroups by 64-slot blocks; every case here is routed to it): within tolerance of
    the oracle and bit-identical to one-vector calls (the VALU kernel), for rows of one block (no
    running sum, no workspace) and of several, ragged 32-row tiles, grids where a workgroup takes
    one tile and several (the two-stage ring), 4-vector launches (3 and 4 vectors), and launches of
    16 + 4 and 16 + 8 vectors; one vector is all zeros (the signs of zero sums must agree too)."""
    t = qvx.Q6_K
    rng = np.random.default_rng(rows + 7 * cols + nvec)
    w = random_weight(t, rows, cols, rng)
    X = rng.standard_normal((nvec, cols)).astype(np.float32)
    X[1] = 0.0
    got = run_gemv(cuda, w, t, X, rows, cols)
    assert max_rel(got, oracle.matmul_f64(w, t, X, nvec, rows, cols)) <= GEMV_TOL
    for v in range(nvec):
        single = run_gemv(cuda, w, t, X[v:v + 1], rows, cols)
        np.testing.assert_array_equal(f32bits(got[v]), f32bits(single[0]))


@pytest.mark.parametrize("rows,cols,nvec", [(4096, 14336, 16), (4096, 14336, 3), (300, 14336, 5), (4099, 14336, 8),
                                             (17, 5120, 2), (64, 4352, 7), (1000, 28672, 8), (33, 4608, 6)])
def test_gemv_q4k_long_row_batched_form_bit_identical(cuda, rows, cols, nvec):
    """Rows too long for the batched form's whole-row fragments (K > 4096) take the long-row form
    (activations converted per super-block by each wave): within tolerance of the oracle and
    bit-identical to one-vector calls, across K splits where waves own one or two super-blocks,
    ragged rows, and more than 16 rows per workgroup (tiles sharing super-blocks)."""
    t = qvx.Q4_K
    rng = np.random.default_rng(rows + 5 * cols + nvec)
    w = random_weight(t, rows, cols, rng)
    X = rng.standard_normal((nvec, cols)).astype(np.float32)
    got = run_gemv(cuda, w, t, X, rows, cols)
    assert max_rel(got, oracle.matmul_f64(w, t, X, nvec, rows, cols)) <= GEMV_TOL
    for v in range(nvec):
        single = run_gemv(cuda, w, t, X[v:v + 1], rows, cols)
        np.testing.assert_array_equal(f32bits(got[v]), f32bits(single[0]))


@pytest.mark.parametrize("rows,cols,nvec", [(1024, 4096, 12), (1000, 4096, 20), (4096, 14336, 23), (100, 8192, 5),
                                             (4099, 14336, 9), (300, 28672, 16), (257, 10240, 7)])
def test_gemv_q4k_split_form_bit_identical(cuda, rows, cols, nvec):
    """The split Q4_K form (K ranges of the one-vector geometry grouped into columns over workgroups,
    range partials summed in order by a second launch; long rows from 5 vectors, small weights from
    12, up to 23): within tolerance of the oracle and bit-identical to one-vector calls, for columns
    of one range (long rows) and of several, 8- and 16-vector launches (16 + 7), ragged tiles,
    workgroups of one tile and of several; one vector is all zeros."""
    t = qvx.Q4_K
    rng = np.random.default_rng(rows + 11 * cols + nvec)
    w = random_weight(t, rows, cols, rng)
    X = rng.standard_normal((nvec, cols)).astype(np.float32)
    X[1] = 0.0
    got = run_gemv(cuda, w, t, X, rows, cols)
    assert max_rel(got, oracle.matmul_f64(w, t, X, nvec, rows, cols)) <= GEMV_TOL
    for v in range(nvec):
        single = run_gemv(cuda, w, t, X[v:v + 1], rows, cols)
        np.testing.assert_array_equal(f32bits(got[v]), f32bits(single[0]))


OTHER_TYPES = [qvx.F16, qvx.BF16, qvx.Q4_1, qvx.Q5_1, qvx.Q8_1]


@pytest.mark.parametrize("t", OTHER_TYPES)
@pytest.mark.parametrize("rows,cols,nvec", [(37, 256, 1), (300, 2048, 3), (1024, 4096, 2)])
def test_gemv_other_dequantizable_types(cuda, t, rows, cols, nvec):
    """Types the reference's qmatmul accepts beyond the integer fast kernels (the float kernel for
    F16 / BF16, the generic kernel for the rest):
    within tolerance of the oracle, batched calls bit-identical to single ones."""
    rng = np.random.default_rng(rows + cols + 13 * t + nvec)
    w = random_weight(t, rows, cols, rng)
    X = rng.standard_normal((nvec, cols)).astype(np.float32)
    got = run_gemv(cuda, w, t, X, rows, cols)
    assert max_rel(got, oracle.matmul_f64(w, t, X, nvec, rows, cols)) <= GEMV_TOL
    for v in range(nvec):
        np.testing.assert_array_equal(f32bits(got[v]), f32bits(run_gemv(cuda, w, t, X[v:v + 1], rows, cols)[0]))


@pytest.mark.parametrize("t", GEMV_TYPES)
def test_gemv_unaligned_weight_uses_generic_path(cuda, t):
    rng = np.random.default_rng(77 + t)
    bs, _ = BLOCK[t]
    rows, cols = 45, 5 * bs  # row pitch not a multiple of 16 for the 32-blocks
    w = random_weight(t, rows, cols, rng)
    X = rng.standard_normal((3, cols)).astype(np.float32)
    ref = oracle.matmul_f64(w, t, X, 3, rows, cols)
    for off in (0, 2, 6):
        got = run_gemv(cuda, w, t, X, rows, cols, offset=off)
        assert max_rel(got, ref) <= GEMV_TOL


FLOAT_TYPES = [qvx.F32, qvx.F16, qvx.BF16]


@pytest.mark.parametrize("t", FLOAT_TYPES)
@pytest.mark.parametrize("rows,cols,nvec", [(4096, 4096, 9), (33, 520, 3), (300, 14336, 5), (17, 32768, 2),
                                             (5, 33280, 2), (1, 8, 1)])
def test_gemv_float_weights(cuda, t, rows, cols, nvec):
    """Unquantised weights on the float kernel: within tolerance of the oracle (fp32 dequant + f64
    dot) and batched calls bit-identical to single ones, across rows that end inside a block of
    chunks, K where the activation budget takes 4, 2 or 1 vectors a launch, and K past it (the
    generic kernel)."""
    rng = np.random.default_rng(rows + cols + 7 * t + nvec)
    w = random_weight(t, rows, cols, rng)
    X = rng.standard_normal((nvec, cols)).astype(np.float32)
    got = run_gemv(cuda, w, t, X, rows, cols)
    assert max_rel(got, oracle.matmul_f64(w, t, X, nvec, rows, cols)) <= GEMV_TOL
    for v in range(nvec):
        np.testing.assert_array_equal(f32bits(got[v]), f32bits(run_gemv(cuda, w, t, X[v:v + 1], rows, cols)[0]))


def test_gemv_f32_weight(cuda):
    rng = np.random.default_rng(4)
    rows, cols = 33, 96
    w = rng.standard_normal(rows * cols).astype(np.float32)
    X = rng.standard_normal((2, cols)).astype(np.float32)
    got = run_gemv(cuda, w.view(np.uint8), qvx.F32, X, rows, cols)
    assert max_rel(got, X.astype(np.float64) @ w.reshape(rows, cols).astype(np.float64).T) <= 1e-5


def test_gemv_zero_cols_writes_zeros(cuda):
    out = cuda.full((5,), 3.0, dtype=cuda.float32, device="cuda")
    rc = qvx.qmatmul(out.data_ptr(), 0, qvx.Q4_K, 0, 5, 0, cuda.cuda.current_stream().cuda_stream)
    assert rc == qvx.OK
    cuda.cuda.synchronize()
    assert np.all(out.cpu().numpy() == 0)


@pytest.mark.parametrize("offset,n", [(0, 5), (1, 7), (3, 9), (2, 1), (1, 4099)])
def test_zero_fill_head_and_tail(cuda, offset, n):
    """cols == 0 zero-fills through the library's zero kernel: vector stores from the first 16-byte
    boundary, single floats before it and after the last whole vector; nothing outside is touched."""
    buf = cuda.full((n + 8,), 3.0, dtype=cuda.float32, device="cuda")
    out = buf[offset:offset + n]
    rc = qvx.qmatmul(out.data_ptr(), 0, qvx.Q4_K, 0, n, 0, cuda.cuda.current_stream().cuda_stream)
    assert rc == qvx.OK
    cuda.cuda.synchronize()
    got = buf.cpu().numpy()
    assert np.all(got[offset:offset + n] == 0)
    assert np.all(got[:offset] == 3.0) and np.all(got[offset + n:] == 3.0)


@pytest.mark.parametrize("t", GEMV_TYPES)
def test_gemv_linearity_full_size(cuda, t):
    """Size-independent property at a BASELINE shape: W(a x + b y) = a Wx + b Wy (fp32 tolerance)."""
    rng = np.random.default_rng(900 + t)
    rows, cols = 14336, 4096
    w = random_weight(t, rows, cols, rng)
    x = rng.standard_normal(cols).astype(np.float32)
    y = rng.standard_normal(cols).astype(np.float32)
    X = np.stack([x, y, (2 * x - 3 * y).astype(np.float32)])
    out = run_gemv(cuda, w, t, X, rows, cols)
    assert max_rel(out[2], 2 * out[0].astype(np.float64) - 3 * out[1]) <= 2 * GEMV_TOL
    assert max_rel(out, oracle.matmul_f64(w, t, X, 3, rows, cols)) <= GEMV_TOL


# Every GEMV shape the BASELINE configs name, with their types and vector counts, on seeded device
# blocks (scales |N(0,1)| * mul as the configs state), against the fp64 oracle.
#   Q8_0 4096x4096 M=1             configs[1]: Q4_0 4096->11008, 11008->4096, M=1
#   Q4_K 4096->14336 / 14336->4096, Q6_K 4096->128256 (lm_head), M in {1, 4, 16}
#   Llama-3-8B Q4_K_M layer (q/o 4096->4096, k/v 4096->1024, gate/up, down; attn_v and
#               ffn_down in Q6_K) and the Q6_K lm_head, M in {1, 8}
BASELINE_GEMV = [
    ("c1 q8_0", qvx.Q8_0, 4096, 4096, (1,), 0.01),
    ("c2 q4_0 up", qvx.Q4_0, 11008, 4096, (1,), 0.02),
    ("c2 q4_0 down", qvx.Q4_0, 4096, 11008, (1,), 0.02),
    ("c3 q4_k gate", qvx.Q4_K, 14336, 4096, (1, 4, 16), 1e-3),
    ("c3 q4_k down", qvx.Q4_K, 4096, 14336, (1, 4, 16), 1e-3),
    ("c3 q6_k lm_head", qvx.Q6_K, 128256, 4096, (1, 4), 1e-3),
    ("c5 q", qvx.Q4_K, 4096, 4096, (1, 8), 1e-3),
    ("c5 k", qvx.Q4_K, 1024, 4096, (1, 8), 1e-3),
    ("c5 v", qvx.Q6_K, 1024, 4096, (1, 8), 1e-3),
    ("c5 down", qvx.Q6_K, 4096, 14336, (1, 8), 1e-3),
]


@pytest.mark.parametrize("name,t,rows,cols,ms,mul", BASELINE_GEMV, ids=[c[0] for c in BASELINE_GEMV])
def test_gemv_baseline_config_shapes(cuda, name, t, rows, cols, ms, mul):
    W = qvx.empty_weight(t, rows, cols)
    qvx.fill_synthetic_t(W, t, rows, cols, seed=rows + cols + t, scale_mul=mul)
    w = W.cpu().numpy()
    for m in ms:
        X = cuda.empty((m, cols), dtype=cuda.float32, device="cuda")
        qvx.fill_normal_t(X, seed=m * 31 + t)
        out = qvx.qmatmul_t(W, t, X, rows, cols)
        cuda.cuda.synchronize()
        ref = oracle.matmul_f64(w, t, X.cpu().numpy(), m, rows, cols)
        assert max_rel(out.cpu().numpy(), ref) <= GEMV_TOL, (name, m)


def test_host_pointer_entry_points(cuda):
    rng = np.random.default_rng(12)
    lib = qvx.lib()
    for t in GEMV_TYPES:
        rows, cols = 40, 1024
        w = random_weight(t, rows, cols, rng)
        X = rng.standard_normal((3, cols)).astype(np.float32)
        out = np.zeros((3, rows), np.float32)
        assert lib.qvx_qmatmul_n_host(out.ctypes.data, w.ctypes.data, t, X.ctypes.data, 3, rows, cols) == qvx.OK
        assert max_rel(out, oracle.matmul_f64(w, t, X, 3, rows, cols)) <= GEMV_TOL
        deq = np.zeros(rows * cols, np.float32)
        assert lib.qvx_dequantize_host(t, w.ctypes.data, deq.ctypes.data, rows * cols) == qvx.OK
        np.testing.assert_array_equal(f32bits(deq), f32bits(oracle.dequantize(t, w, rows * cols)))
        row = np.zeros(cols, np.float32)
        assert lib.qvx_dequant_row_host(w.ctypes.data, t, cols, 7, row.ctypes.data) == qvx.OK
        np.testing.assert_array_equal(f32bits(row), f32bits(deq[7 * cols:8 * cols]))


# ---- GEMM ----------------------------------------------------------------------------------------

@pytest.mark.parametrize("variant", [qvx.GEMM_BF16, qvx.GEMM_F16, qvx.GEMM_I8])
@pytest.mark.parametrize("M,rows,cols", [(128, 512, 1024), (200, 300, 768), (512, 1024, 4096), (37, 256, 256)])
def test_gemm_q4k_parity(cuda, variant, M, rows, cols):
    rng = np.random.default_rng(M + rows + cols + variant)
    t = qvx.Q4_K
    w = random_weight(t, rows, cols, rng, scale=0.002)
    X16 = (rng.standard_normal((M, cols)) * 0.5).astype(np.float16)
    X = dev(cuda, X16.view(np.uint16))
    out = qvx.qgemm_t(dev(cuda, w), t, X, rows, cols, variant)
    cuda.cuda.synchronize()
    ref = oracle.matmul_f64(w, t, X16.astype(np.float32), M, rows, cols)
    assert max_rel(out.cpu().numpy(), ref) <= GEMM_TOL


@pytest.mark.parametrize("variant", [qvx.GEMM_BF16, qvx.GEMM_F16, qvx.GEMM_I8])
@pytest.mark.parametrize("offset", [0, 1, 3])
def test_gemm_split_k_overwrites_stale_output(cuda, variant, offset):
    """M = 128 splits K across workgroups whose partial tiles the last split of each tile sums and
    stores: NaN left in the output buffer never leaks into the result, at any float offset, and
    nothing outside it is written."""
    rng = np.random.default_rng(77 + 10 * variant + offset)
    t, M, rows, cols = qvx.Q4_K, 128, 512, 1024
    w = random_weight(t, rows, cols, rng, scale=0.002)
    X16 = (rng.standard_normal((M, cols)) * 0.5).astype(np.float16)
    X, W = dev(cuda, X16.view(np.uint16)), dev(cuda, w)
    buf = cuda.full((M * rows + 8,), float("nan"), dtype=cuda.float32, device="cuda")
    out = buf[offset:offset + M * rows]
    rc = qvx.lib().qvx_qgemm_f16(out.data_ptr(), W.data_ptr(), t, X.data_ptr(), M, rows, cols, variant,
                                 cuda.cuda.current_stream().cuda_stream)
    assert rc == qvx.OK
    cuda.cuda.synchronize()
    got = buf.cpu().numpy()
    ref = oracle.matmul_f64(w, t, X16.astype(np.float32), M, rows, cols)
    assert np.isfinite(got[offset:offset + M * rows]).all()
    assert max_rel(got[offset:offset + M * rows].reshape(M, rows), ref) <= GEMM_TOL
    assert np.isnan(got[:offset]).all() and np.isnan(got[offset + M * rows:]).all()


@pytest.mark.parametrize("t,variant", [(qvx.Q4_K, qvx.GEMM_BF16), (qvx.Q4_K, qvx.GEMM_F16), (qvx.Q4_K, qvx.GEMM_I8),
                                       (qvx.Q6_K, qvx.GEMM_BF16), (qvx.Q6_K, qvx.GEMM_F16)])
@pytest.mark.parametrize("M,rows,cols", [(128, 14336, 4096), (37, 2048, 4096), (300, 4096, 14336)])
def test_gemm_split_k_is_deterministic(cuda, t, variant, M, rows, cols):
    """Shapes whose grid is smaller than the chip split K; the split that finishes a tile last adds
    the partial tiles in split order 0, 1, ..., so repeated calls (whichever split finishes first)
    give the same bits, and the result stays within the GEMM tolerance of the fp64 oracle on a
    slice of rows (bf16 / fp16 variants)."""
    if t == qvx.Q4_K:
        plan = qvx.qgemm_plan_q4k(M, rows, cols)
        assert variant == qvx.GEMM_I8 or plan[0]["splits"] > 1
    W = qvx.empty_weight(t, rows, cols)
    qvx.fill_synthetic_t(W, t, rows, cols, seed=31 + M + variant, scale_mul=1e-3)
    X = cuda.empty((M, cols), dtype=cuda.float16, device="cuda")
    qvx.fill_normal_t(X, seed=32 + M, mul=0.5)
    runs = [qvx.qgemm_t(W, t, X, rows, cols, variant).cpu().numpy() for _ in range(3)]
    for r in runs[1:]:
        np.testing.assert_array_equal(r.view(np.uint32), runs[0].view(np.uint32))
    idx = np.union1d(np.arange(0, rows, 97), [rows - 1])
    rb = qvx.row_bytes(t, cols)
    Wd = oracle.dequantize(t, W.cpu().numpy().reshape(rows, rb)[idx].reshape(-1), len(idx) * cols)
    ref = X.cpu().numpy().astype(np.float64) @ Wd.reshape(len(idx), cols).astype(np.float64).T
    if variant != qvx.GEMM_I8:  # the Q8 arithmetic has its own oracle test
        assert max_rel(runs[0][:, idx], ref) <= GEMM_TOL


@pytest.mark.parametrize("t", [qvx.Q4_K, qvx.Q6_K])
def test_gemm_split_k_concurrent_streams(cuda, t):
    """K-split GEMMs issued on two streams at once, each call with its own pool workspace for the
    partial tiles and counters, into distinct outputs: every output is bit-identical to the same
    call made alone (overlapping calls on one device are safe for distinct outputs)."""
    M, rows, cols = 128, 2048, 4096
    W = qvx.empty_weight(t, rows, cols)
    qvx.fill_synthetic_t(W, t, rows, cols, seed=71, scale_mul=1e-3)
    Xs = [cuda.empty((M, cols), dtype=cuda.float16, device="cuda") for _ in range(2)]
    for i, X in enumerate(Xs):
        qvx.fill_normal_t(X, seed=72 + i, mul=0.5)
    lib = qvx.lib()
    cuda.cuda.synchronize()
    alone = []
    for X in Xs:
        Y = cuda.empty((M, rows), dtype=cuda.float32, device="cuda")
        assert lib.qvx_qgemm_f16(Y.data_ptr(), W.data_ptr(), t, X.data_ptr(), M, rows, cols, qvx.GEMM_BF16,
                                 cuda.cuda.current_stream().cuda_stream) == qvx.OK
        cuda.cuda.synchronize()
        alone.append(Y.cpu().numpy())
    streams = [cuda.cuda.Stream(), cuda.cuda.Stream()]
    outs = [[cuda.full((M, rows), float("nan"), dtype=cuda.float32, device="cuda") for _ in range(6)]
            for _ in range(2)]
    cuda.cuda.synchronize()
    for k in range(6):
        for i in range(2):
            assert lib.qvx_qgemm_f16(outs[i][k].data_ptr(), W.data_ptr(), t, Xs[i].data_ptr(), M, rows, cols,
                                     qvx.GEMM_BF16, streams[i].cuda_stream) == qvx.OK
    cuda.cuda.synchronize()
    for i in range(2):
        for k in range(6):
            np.testing.assert_array_equal(outs[i][k].cpu().numpy().view(np.uint32), alone[i].view(np.uint32))


def test_gemm_split_k_counters_reused_across_calls(cuda):
    """Calls that may allocate take their K split's tile counters from a block the stream keeps,
    cleared once: every launch leaves the counters it used at zero.  K-split calls of different
    tile counts and kernels (the Q4_K and Q6_K raw-block GEMMs, the 16-bit GEMM behind Q8_0 / Q4_0),
    fp16 and bf16, interleaved on one stream for three rounds and then on a new stream, give the
    first round's bits every time (a counter left non-zero would make a later tile's last split
    skip its sum, or sum too early)."""
    cases = [(qvx.Q4_K, qvx.GEMM_F16, 128, 14336, 4096), (qvx.Q6_K, qvx.GEMM_F16, 300, 4096, 14336),
             (qvx.Q4_K, qvx.GEMM_BF16, 37, 2048, 4096), (qvx.Q8_0, qvx.GEMM_BF16, 128, 4096, 4096),
             (qvx.Q4_K, qvx.GEMM_F16, 200, 1024, 4096), (qvx.Q6_K, qvx.GEMM_BF16, 128, 1024, 4096),
             (qvx.Q4_0, qvx.GEMM_F16, 96, 4096, 11008)]
    lib = qvx.lib()
    data = []
    for i, (t, variant, M, rows, cols) in enumerate(cases):
        W = qvx.empty_weight(t, rows, cols)
        qvx.fill_synthetic_t(W, t, rows, cols, seed=90 + i, scale_mul=1e-3)
        X = cuda.empty((M, cols), dtype=cuda.float16, device="cuda")
        qvx.fill_normal_t(X, seed=95 + i, mul=0.5)
        data.append((W, X))
    assert qvx.qgemm_plan_q4k(128, 14336, 4096)[0]["splits"] > 1  # the premise: these calls split K
    cuda.cuda.synchronize()

    def round_on(stream):
        outs = []
        for (t, variant, M, rows, cols), (W, X) in zip(cases, data):
            Y = cuda.full((M, rows), float("nan"), dtype=cuda.float32, device="cuda")
            assert lib.qvx_qgemm_f16(Y.data_ptr(), W.data_ptr(), t, X.data_ptr(), M, rows, cols, variant,
                                     stream.cuda_stream) == qvx.OK
            outs.append(Y)
        stream.synchronize()
        return [o.cpu().numpy() for o in outs]

    cur = cuda.cuda.current_stream()
    first = round_on(cur)
    for r in range(2):
        for i, got in enumerate(round_on(cur)):
            np.testing.assert_array_equal(got.view(np.uint32), first[i].view(np.uint32), err_msg=f"round {r} case {i}")
    fresh = cuda.cuda.Stream()
    for i, got in enumerate(round_on(fresh)):
        np.testing.assert_array_equal(got.view(np.uint32), first[i].view(np.uint32), err_msg=f"new stream case {i}")
    for i, (t, variant, M, rows, cols) in enumerate(cases):
        assert np.isfinite(first[i]).all(), i


GROUP_CASES = [
    # the decoder's q / k / v (Q6_K v) and gate / up of Llama-3-8B
    ("qkv", 4096, [(qvx.Q4_K, 4096), (qvx.Q4_K, 1024), (qvx.Q6_K, 1024)]),
    ("gate_up", 4096, [(qvx.Q4_K, 14336), (qvx.Q4_K, 14336)]),
    # two conversion tasks a thread (K = 16384), a Q6_K member of 8 rows a group
    ("long_k", 16384, [(qvx.Q6_K, 4096), (qvx.Q4_K, 1000)]),
    # ragged row counts (a Q6_K member of 5 rows a group), four Q4_K members
    ("ragged", 2048, [(qvx.Q4_K, 777), (qvx.Q6_K, 20000), (qvx.Q4_K, 17), (qvx.Q4_K, 1), (qvx.Q4_K, 300)]),
    # a Q6_K member walking its rows in chunks (10 rows a group)
    ("chunked", 2048, [(qvx.Q6_K, 40000), (qvx.Q4_K, 64)]),
    # K = 2304: 72 Q6_K slots in groups of 128 lanes, the padding lanes mirroring the last slot
    ("padded", 2304, [(qvx.Q6_K, 300), (qvx.Q4_K, 64)]),
    # outside the grouped kernel (two Q6_K members; five Q4_K; a Q8_0 member; a Q6_K row of 448
    # slots, whose VALU workgroup is not 1024 threads): member by member
    ("two_q6k", 4096, [(qvx.Q6_K, 1024), (qvx.Q6_K, 512)]),
    ("q6k_k14336", 14336, [(qvx.Q4_K, 256), (qvx.Q6_K, 512)]),
    ("five_q4k", 1024, [(qvx.Q4_K, 64)] * 5),
    ("q8_0", 4096, [(qvx.Q4_K, 512), (qvx.Q8_0, 512)]),
    # a member with no rows computes nothing
    ("empty_member", 4096, [(qvx.Q4_K, 256), (qvx.Q6_K, 0), (qvx.Q6_K, 96)]),
]


@pytest.mark.parametrize("norm", [False, True], ids=["plain", "rmsnorm"])
@pytest.mark.parametrize("name,cols,members", GROUP_CASES, ids=[c[0] for c in GROUP_CASES])
def test_qmatmul_group_matches_single_calls(cuda, name, cols, members, norm):
    """qvx_qmatmul_group: each member's output bit-identical to its own qvx_qmatmul (with a norm: its
    own qvx_qmatmul_n_rmsnorm), whether the members run as one launch or one by one; a member's
    neighbours' rows stay untouched."""
    torch = cuda
    x = torch.empty(cols, dtype=torch.float32, device="cuda")
    qvx.fill_normal_t(x, seed=81, mul=1.0)
    nw = torch.empty(cols, dtype=torch.float32, device="cuda")
    qvx.fill_normal_t(nw, seed=82, mul=0.2)
    nw.add_(1.0)
    eps = 1e-5
    ws, outs, refs = [], [], []
    for i, (t, rows) in enumerate(members):
        w = qvx.empty_weight(t, max(rows, 1), cols)
        qvx.fill_synthetic_t(w, t, max(rows, 1), cols, seed=90 + i, scale_mul=1e-3)
        ws.append(w)
        outs.append(torch.full((rows + 16,), float("nan"), dtype=torch.float32, device="cuda"))
        r = torch.empty(max(rows, 1), dtype=torch.float32, device="cuda")
        if norm:
            assert qvx.qmatmul_n_rmsnorm(r.data_ptr(), w.data_ptr(), t, x.data_ptr(), nw.data_ptr(), eps, 1, rows,
                                         cols) == qvx.OK
        else:
            assert qvx.qmatmul(r.data_ptr(), w.data_ptr(), t, x.data_ptr(), rows, cols) == qvx.OK
        refs.append(r)
    torch.cuda.synchronize()
    for _ in range(2):
        rc = qvx.qmatmul_group([o.data_ptr() for o in outs], [w.data_ptr() for w in ws], [t for t, _ in members],
                               [r for _, r in members], x.data_ptr(), cols, norm_w=nw.data_ptr() if norm else 0,
                               eps=eps)
        assert rc == qvx.OK
        torch.cuda.synchronize()
        for i, ((t, rows), o, r) in enumerate(zip(members, outs, refs)):
            assert torch.equal(o[:rows].view(torch.int32), r[:rows].view(torch.int32)), (name, i)
            assert torch.isnan(o[rows:]).all(), (name, i)


def test_qmatmul_group_matches_oracle(cuda):
    """The grouped q / k / v launch against the oracle (a slice of rows of each member)."""
    torch = cuda
    cols = 4096
    members = [(qvx.Q4_K, 4096), (qvx.Q4_K, 1024), (qvx.Q6_K, 1024)]
    x = torch.empty(cols, dtype=torch.float32, device="cuda")
    qvx.fill_normal_t(x, seed=83, mul=1.0)
    ws = []
    for i, (t, rows) in enumerate(members):
        w = qvx.empty_weight(t, rows, cols)
        qvx.fill_synthetic_t(w, t, rows, cols, seed=95 + i, scale_mul=1e-3)
        ws.append(w)
    outs = [torch.empty(rows, dtype=torch.float32, device="cuda") for _, rows in members]
    assert qvx.qmatmul_group([o.data_ptr() for o in outs], [w.data_ptr() for w in ws], [t for t, _ in members],
                             [r for _, r in members], x.data_ptr(), cols) == qvx.OK
    torch.cuda.synchronize()
    xs = x.cpu().numpy()[None, :]
    for (t, rows), w, o in zip(members, ws, outs):
        rb = qvx.row_bytes(t, cols)
        r0, nr = rows - 40, 40
        ref = oracle.matmul_f64(w[r0 * rb:(r0 + nr) * rb].cpu().numpy(), t, xs, 1, nr, cols)
        assert max_rel(o[r0:].cpu().numpy()[None, :], ref) <= 1e-3, t


DEQUANT_GEMM_TYPES = [qvx.Q6_K, qvx.Q8_0, qvx.Q4_0, qvx.Q5_0, qvx.Q5_K, qvx.Q4_1, qvx.Q5_1, qvx.Q8_1,
                      qvx.F16, qvx.BF16, qvx.F32]


@pytest.mark.parametrize("t", DEQUANT_GEMM_TYPES)
@pytest.mark.parametrize("variant", [qvx.GEMM_BF16, qvx.GEMM_F16])
@pytest.mark.parametrize("M,rows,cols", [(128, 512, 1024), (37, 300, 256), (37, 300, 2304)])
def test_gemm_other_types_parity(cuda, t, variant, M, rows, cols):
    """The weight types other than Q4_K (Q6_K on its raw-block MFMA kernels: k_qgemm_q6k8 at cols 512 and
    1024, k_qgemm_deq at the odd block counts of cols 256 and 2304; the rest dequantised to 16 bits for
    the plain MFMA GEMM), within the GEMM tolerance of the fp64 oracle, on 128 x 512 x 1024, 37 x 300 x
    256 (ragged tiles in M and N) and 37 x 300 x 2304 (K split into ranges of an odd length)."""
    rng = np.random.default_rng(M + rows + cols + 3 * t + variant)
    w = random_weight(t, rows, cols, rng, scale=0.002)
    X16 = (rng.standard_normal((M, cols)) * 0.5).astype(np.float16)
    out = qvx.qgemm_t(dev(cuda, w), t, dev(cuda, X16.view(np.uint16)), rows, cols, variant)
    cuda.cuda.synchronize()
    ref = oracle.matmul_f64(w, t, X16.astype(np.float32), M, rows, cols)
    assert max_rel(out.cpu().numpy(), ref) <= GEMM_TOL


@pytest.mark.parametrize("variant", [qvx.GEMM_BF16, qvx.GEMM_F16])
@pytest.mark.parametrize("M,rows,cols", [(37, 300, 512), (200, 300, 2560), (130, 520, 3072), (1, 256, 1024),
                                         (300, 2100, 2048)])
def test_gemm_q6k_pipeline_shapes(cuda, variant, M, rows, cols):
    """Q6_K with an even number of blocks a row runs on the Q4_K kernel's pipeline (each super-block
    of the tile's rows staged whole, dequantised in registers): ragged token and row tiles, K of one
    to six super-block pairs, one K range (37 x 300 x 512, M = 1), two splits of five super-blocks
    (200 x 300 x 2560) and two of six or four (130 x 520 x 3072, 300 x 2100 x 2048), against the
    fp64 oracle.  The same call on a copy of W two bytes off its dword alignment, which the staged
    copies cannot take, goes to the 16-bit dequantiser and the plain MFMA GEMM and meets the same
    bound."""
    rng = np.random.default_rng(M + rows + cols + variant)
    t = qvx.Q6_K
    w = random_weight(t, rows, cols, rng, scale=0.002)
    X16 = (rng.standard_normal((M, cols)) * 0.5).astype(np.float16)
    X = dev(cuda, X16.view(np.uint16))
    ref = oracle.matmul_f64(w, t, X16.astype(np.float32), M, rows, cols)
    out = qvx.qgemm_t(dev(cuda, w), t, X, rows, cols, variant)
    cuda.cuda.synchronize()
    assert max_rel(out.cpu().numpy(), ref) <= GEMM_TOL
    buf = cuda.zeros(w.size + 16, dtype=cuda.uint8, device="cuda")
    buf[2:2 + w.size] = cuda.from_numpy(w.reshape(-1).view(np.uint8)).to("cuda")
    out2 = cuda.full((M, rows), float("nan"), dtype=cuda.float32, device="cuda")
    rc = qvx.lib().qvx_qgemm_f16(out2.data_ptr(), buf.data_ptr() + 2, t, X.data_ptr(), M, rows, cols, variant,
                                 cuda.cuda.current_stream().cuda_stream)
    assert rc == qvx.OK
    cuda.cuda.synchronize()
    assert max_rel(out2.cpu().numpy(), ref) <= GEMM_TOL


@pytest.mark.parametrize("t", [qvx.Q8_0, qvx.Q4_0, qvx.Q5_1])
def test_gemm_32_blocks_odd_slices(cuda, t):
    """32-element block types at cols = 320 and cols = 96 (not a multiple of 64), against the
    oracle."""
    rng = np.random.default_rng(70 + t)
    for M, rows, cols in ((45, 260, 320), (9, 40, 96)):
        w = random_weight(t, rows, cols, rng, scale=0.002)
        X16 = (rng.standard_normal((M, cols)) * 0.5).astype(np.float16)
        ref = oracle.matmul_f64(w, t, X16.astype(np.float32), M, rows, cols)
        for variant in (qvx.GEMM_BF16, qvx.GEMM_F16):
            out = qvx.qgemm_t(dev(cuda, w), t, dev(cuda, X16.view(np.uint16)), rows, cols, variant)
            cuda.cuda.synchronize()
            assert max_rel(out.cpu().numpy(), ref) <= GEMM_TOL, (M, rows, cols, variant)


def _round16(v32, bf16):
    """fp32 -> fp16 or bf16 bits, round to nearest even (finite inputs)."""
    if not bf16:
        return v32.astype(np.float16).view(np.uint16)
    u = v32.view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


@pytest.mark.parametrize("t,cols", [(t, 512) for t in DEQUANT_GEMM_TYPES] + [(qvx.Q6_K, 2304)])
@pytest.mark.parametrize("variant", [qvx.GEMM_BF16, qvx.GEMM_F16])
@pytest.mark.parametrize("src_offset", [0, 2])
def test_gemm_dequant16_bit_exact(cuda, t, cols, variant, src_offset):
    """The 16-bit weight operand of the GEMM, read back exactly: with X the identity (M = cols),
    out[m, r] = W16[r, m] (one nonzero product per sum, exact in fp32), which must equal the oracle's
    dequantised fp32 value rounded once to fp16 / bf16.  Which kernel builds the operand: Q6_K at
    cols 512 (an even number of blocks a row) on k_qgemm_q6k8, at cols 2304 (an odd number) on the
    dequantising MFMA kernel k_qgemm_deq, in both cases in registers or LDS from the raw blocks;
    src_offset 2 moves the blocks off 4-byte alignment, which both decline, and every other type always
    goes through the 16-bit dequantiser (qvx_dequantize16's kernels) and the plain MFMA GEMM.  Zeros are
    compared without their sign."""
    if t == qvx.F32 and src_offset:
        pytest.skip("fp32 weights are 4-byte values: a 2-byte offset is not a layout they come in")
    rng = np.random.default_rng(5 * t + variant + src_offset + cols)
    rows = 300
    w = random_weight(t, rows, cols, rng, scale=0.002)
    raw = cuda.zeros(w.size + 16, dtype=cuda.uint8, device="cuda")
    raw[src_offset:src_offset + w.size].copy_(cuda.from_numpy(w))
    X = dev(cuda, np.eye(cols, dtype=np.float16).view(np.uint16))
    out = cuda.empty((cols, rows), dtype=cuda.float32, device="cuda")
    rc = qvx.lib().qvx_qgemm_f16(out.data_ptr(), raw.data_ptr() + src_offset, t, X.data_ptr(), cols, rows, cols,
                                 variant, cuda.cuda.current_stream().cuda_stream)
    assert rc == qvx.OK
    cuda.cuda.synchronize()
    got = out.cpu().numpy().T.copy()  # [rows, cols]
    want16 = _round16(oracle.dequantize(t, w, rows * cols).astype(np.float32), variant == qvx.GEMM_BF16)
    want = (want16.astype(np.uint32) << 16).view(np.float32) if variant == qvx.GEMM_BF16 else \
        want16.view(np.float16).astype(np.float32)
    # + 0.0: a sum that holds one -0 product and +0 products is +0, so zeros compare without sign
    np.testing.assert_array_equal(f32bits(got.reshape(-1) + np.float32(0)), f32bits(want.reshape(-1) + np.float32(0)))


@pytest.mark.parametrize("t", [qvx.F16, qvx.BF16, qvx.F32])
def test_gemm_float_weights_ragged_tail(cuda, t):
    """rows * cols not a multiple of 8: the dequantiser's vector kernel takes the whole groups of 8
    and the scalar kernel the tail."""
    rng = np.random.default_rng(5 + t)
    M, rows, cols = 5, 3, 260
    w = random_weight(t, rows, cols, rng, scale=0.002)
    X16 = (rng.standard_normal((M, cols)) * 0.5).astype(np.float16)
    ref = oracle.matmul_f64(w, t, X16.astype(np.float32), M, rows, cols)
    for variant in (qvx.GEMM_BF16, qvx.GEMM_F16):
        out = qvx.qgemm_t(dev(cuda, w), t, dev(cuda, X16.view(np.uint16)), rows, cols, variant)
        cuda.cuda.synchronize()
        assert max_rel(out.cpu().numpy(), ref) <= GEMM_TOL


def test_gemm_q6k_ffn_down_shape(cuda):
    """The Q4_K_M model's Q6_K ffn_down (14336 -> 4096) at M = 64 on k_qgemm_q6k8 (K = 14336 is a
    whole number of super-block pairs; 128-token tiles, K split 8 ways), and the int8 variant refused
    for it."""
    t, M, rows, cols = qvx.Q6_K, 64, 4096, 14336
    W = qvx.empty_weight(t, rows, cols)
    qvx.fill_synthetic_t(W, t, rows, cols, seed=41, scale_mul=1e-3)
    X = cuda.empty((M, cols), dtype=cuda.float16, device="cuda")
    qvx.fill_normal_t(X, seed=42, mul=0.5)
    ref = oracle.matmul_f64(W.cpu().numpy(), t, X.cpu().numpy().astype(np.float32), M, rows, cols)
    for variant in (qvx.GEMM_BF16, qvx.GEMM_F16):
        out = qvx.qgemm_t(W, t, X, rows, cols, variant)
        cuda.cuda.synchronize()
        assert max_rel(out.cpu().numpy(), ref) <= GEMM_TOL
    with pytest.raises(qvx.QvxError):
        qvx.qgemm_t(W, t, X, rows, cols, qvx.GEMM_I8)


def test_gemm_q4k_config4_shape(cuda):
    """BASELINE config 4 (Q4_K 4096 -> 14336, M = 128) against the fp64 oracle."""
    rng = np.random.default_rng(2024)
    t, M, rows, cols = qvx.Q4_K, 128, 14336, 4096
    W = qvx.empty_weight(t, rows, cols)
    qvx.fill_synthetic_t(W, t, rows, cols, seed=31, scale_mul=1e-3)
    X = cuda.empty((M, cols), dtype=cuda.float16, device="cuda")
    qvx.fill_normal_t(X, seed=32, mul=0.5)
    for variant in (qvx.GEMM_BF16, qvx.GEMM_F16, qvx.GEMM_I8):
        out = qvx.qgemm_t(W, t, X, rows, cols, variant)
        cuda.cuda.synchronize()
        w = W.cpu().numpy()
        ref = oracle.matmul_f64(w, t, X.cpu().numpy().astype(np.float32), M, rows, cols)
        assert max_rel(out.cpu().numpy(), ref) <= GEMM_TOL


@pytest.mark.parametrize("M,rows,cols", [(128, 512, 1024), (200, 300, 768), (37, 256, 256), (640, 768, 2048)])
def test_gemm_i8_matches_quantized_oracle(cuda, M, rows, cols):
    """The int8 variant computes sum_b sx_b * sum_k q_k * w_k exactly up to fp32 rounding: compare with
    the oracle's Q8 quantiser and bit-exact dequant, multiplied in fp64 (tolerance 1e-4)."""
    rng = np.random.default_rng(M * 7 + rows + cols)
    t = qvx.Q4_K
    w = random_weight(t, rows, cols, rng, scale=0.002)
    X16 = (rng.standard_normal((M, cols)) * 0.5).astype(np.float16)
    X16[1, 32:64] = 0  # an all-zero block: scale 0
    out = qvx.qgemm_t(dev(cuda, w), t, dev(cuda, X16.view(np.uint16)), rows, cols, qvx.GEMM_I8)
    cuda.cuda.synchronize()
    q, s, _ = oracle.quantize_q8_act(X16.astype(np.float32))
    Xq = q.astype(np.float64) * np.repeat(s.astype(np.float64), 32, axis=1)
    Wd = oracle.dequantize(t, w, rows * cols).reshape(rows, cols).astype(np.float64)
    ref = Xq @ Wd.T
    assert max_rel(out.cpu().numpy(), ref) <= 1e-4


def test_quantize_act_q8_matches_oracle(cuda):
    rng = np.random.default_rng(8)
    M, K = 19, 512
    X16 = (rng.standard_normal((M, K)) * 0.5).astype(np.float16)
    X16[3, 64:96] = 0
    X = dev(cuda, X16.view(np.uint16))
    q = cuda.empty((M, K), dtype=cuda.int8, device="cuda")
    s = cuda.empty((M, K // 32), dtype=cuda.float32, device="cuda")
    qs = cuda.empty((M, K // 32), dtype=cuda.int32, device="cuda")
    rc = qvx.lib().qvx_quantize_act_q8(X.data_ptr(), M, K, q.data_ptr(), s.data_ptr(), qs.data_ptr(),
                                       cuda.cuda.current_stream().cuda_stream)
    assert rc == qvx.OK
    cuda.cuda.synchronize()
    oq, os_, oqs = oracle.quantize_q8_act(X16.astype(np.float32))
    np.testing.assert_array_equal(q.cpu().numpy(), oq)
    np.testing.assert_array_equal(f32bits(s.cpu().numpy()), f32bits(os_))
    np.testing.assert_array_equal(qs.cpu().numpy(), oqs)


# ---- synthetic data generator ---------------------------------------------------------------------

def test_synthetic_blocks_are_well_formed(cuda):
    for t, mul in ((qvx.Q8_0, 0.01), (qvx.Q4_0, 0.02), (qvx.Q4_K, 1e-3), (qvx.Q5_K, 1e-3), (qvx.Q6_K, 1e-3)):
        rows, cols = 64, 4096
        W = qvx.empty_weight(t, rows, cols)
        qvx.fill_synthetic_t(W, t, rows, cols, seed=5, scale_mul=mul)
        W2 = qvx.empty_weight(t, rows, cols)
        qvx.fill_synthetic_t(W2, t, rows, cols, seed=5, scale_mul=mul)
        cuda.cuda.synchronize()
        a, b = W.cpu().numpy(), W2.cpu().numpy()
        np.testing.assert_array_equal(a, b)  # deterministic
        deq = oracle.dequantize(t, a, rows * cols)
        assert np.all(np.isfinite(deq))
        bs, bb = BLOCK[t]
        blk = a.reshape(-1, bb)
        off = 208 if t == qvx.Q6_K else 0
        d = blk[:, off:off + 2].copy().view(np.float16).astype(np.float64).ravel()
        assert np.all(d >= 0) and 0.5 * mul < d.mean() < 1.1 * mul  # E|N(0,1)| = 0.798
        if t == qvx.Q8_0:
            q = blk[:, 2:].view(np.int8)
            assert q.min() == -127 and q.max() == 127


def test_bench_read_stores_only_on_the_pattern(cuda):
    """The bare-read helper stores nothing for ordinary data and 1 when a word holds the pattern."""
    buf = cuda.zeros(1 << 20, dtype=cuda.uint8, device="cuda")
    flag = cuda.zeros(1, dtype=cuda.int32, device="cuda")
    s = cuda.cuda.current_stream().cuda_stream
    assert qvx.lib().qvx_bench_read(buf.data_ptr(), buf.numel(), flag.data_ptr(), s) == qvx.OK
    cuda.cuda.synchronize()
    assert int(flag.item()) == 0
    buf.view(cuda.int32)[4096:4100] = 0x5A17C0DE
    assert qvx.lib().qvx_bench_read(buf.data_ptr(), buf.numel(), flag.data_ptr(), s) == qvx.OK
    cuda.cuda.synchronize()
    assert int(flag.item()) == 1
