/*
 * qvx.h -- C ABI of the MI355X (gfx950) GGUF quantized-matmul engine (libqvx.so).
 *
 * The engine computes the QorVix weight x activation operator on the GPU:
 *   out[v, r] = sum_k dequant(W)[r, k] * X[v, k]
 * with W in raw GGUF block layout (row r starts at r * (cols / blockSize) * typeSize bytes),
 * X fp32 [n_vec, cols] row-major and out fp32 [n_vec, rows] row-major -- the reference's
 * qmatmul / qmatmulN contract (runtime/include/qorvix/runtime/qmatmul.hpp:14-36).
 *
 * Conventions
 *  - `type` is the raw on-disk ggml type id (Q4_0 = 2, Q8_0 = 8, Q4_K = 12, Q6_K = 14, F32 = 0, ...).
 *  - Every call returns QVX_OK (0) or a negative QVX_E_* code.  All argument checks run before any
 *    device work, so `out` is untouched on a check's failure (QVX_E_TYPE, _SHAPE, _NVEC, _NULL,
 *    _VARIANT, _RANGE) -- the reference's `false` cases map one for one:
 *      unknown / unsupported type        -> QVX_E_TYPE   (qmatmul.cpp:30-31)
 *      blockSize > 256 or cols % bs != 0 -> QVX_E_SHAPE  (qmatmul.cpp:32-33, :70-72)
 *      n_vec <= 0                        -> QVX_E_NVEC   (qmatmul.cpp:66)
 *    rows <= 0 is a successful no-op and cols == 0 writes zeros, as the reference's loops do.
 *    QVX_E_HIP reports a runtime failure after the checks passed (a launch the runtime refused, a
 *    failed allocation or copy); calls that issue several launches (a batch in chunks of vectors, a
 *    GEMM in panels) may then have written part of `out`, whose contents are unspecified.
 *  - Device entry points take device pointers and a hipStream_t passed as `void*` (NULL = the
 *    null stream).  They are asynchronous and stream-ordered, like the CUDA backend's matmulS
 *    launch (cuda/src/cuda_backend.cu:1534-1542).  They allocate no device memory, except
 *    qvx_qgemm_f16, qvx_gemm16, the many-vector form of qvx_qmatmul_n and the unfused norm route,
 *    which take stream-ordered temporaries (the converted activations, the partial tiles of a K
 *    split, or the dequantised weight) from a memory pool the library owns per device.  Each stream
 *    keeps its last temporary for its next call (no pool call between back-to-back calls), and a
 *    block of K-split tile counters (64 KiB or more, cleared once, left zero by every launch) for
 *    the life of the process, so a caller that destroys a stream must first let the qvx calls
 *    issued to it finish (synchronize the stream): a new stream may be handed the same handle.
 *  - Entry points ending in _host take host pointers and are synchronous: the exact calling
 *    convention of the reference's CPU operator, for a CPU-side drop-in.
 *  - Calls that overlap on one device are safe for distinct outputs; the library holds no
 *    mutable per-call state (the GEMM temporaries are per call, or per stream, and stream-ordered).
 */
#ifndef QVX_H
#define QVX_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define QVX_OK 0
#define QVX_E_TYPE (-1)    /* unknown ggml type, or one this engine does not compute */
#define QVX_E_SHAPE (-2)   /* cols not a multiple of the block size, block size > 256, bad M/K */
#define QVX_E_NVEC (-3)    /* n_vec <= 0 */
#define QVX_E_NULL (-4)    /* a required pointer is NULL */
#define QVX_E_HIP (-5)     /* the HIP runtime reported an error (launch, copy, allocation) */
#define QVX_E_VARIANT (-6) /* unknown GEMM variant */
#define QVX_E_RANGE (-7)   /* row index out of range, n not a whole number of blocks, size overflow */
#define QVX_E_STATE (-8)   /* a plan launched before qvx_plan_instantiate, or changed after it */
#define QVX_E_FORMAT (-9)  /* malformed GGUF data (qvx_gguf_last_error() says what) */
#define QVX_E_IO (-10)     /* a file could not be opened or mapped */
#define QVX_E_LIB (-11)    /* a runtime library the call needs is missing or failed (no current call needs one) */

/* GEMM variants for qvx_qgemm_f16 */
#define QVX_GEMM_BF16 0 /* X rounded to bf16; raw weight blocks staged in LDS, dequantised to bf16; bf16 MFMA */
#define QVX_GEMM_I8 1   /* X quantised per 32 to int8 (Q8), weight quants as int8, int8 MFMA */
#define QVX_GEMM_F16 2  /* X kept fp16; raw weight blocks staged in LDS, dequantised to fp16; fp16 MFMA */

/* Version string of the engine, e.g. "qvx 0.1 gfx950". */
const char* qvx_version(void);

/* Message of a QVX_E_* code. */
const char* qvx_strerror(int code);

/* 1 if qvx_qmatmul / qvx_qmatmul_n compute `type` (qmatmul.cpp:24-26, qmatmulSupports): every
 * type the reference dequantises (F32, F16, BF16, Q8_0, Q8_1, Q4_0, Q4_1, Q5_0, Q5_1, Q4_K, Q5_K,
 * Q6_K).  Q8_0 / Q4_0 / Q5_0 / Q4_K / Q5_K / Q6_K run on the integer fast kernels, F32 / F16 /
 * BF16 on the float kernel, Q8_1 / Q4_1 / Q5_1 and unaligned weights on a generic kernel.
 * qvx_qgemm_f16 computes the same types. */
int qvx_supports(uint32_t type);

/* 1 if qvx_dequantize handles `type` (dequant.cpp:257-275, canDequantize). */
int qvx_can_dequantize(uint32_t type);

/* Elements per block and bytes per block of a ggml type; 0 if unknown (gguf_types.cpp:49-54). */
int qvx_type_traits(uint32_t type, uint32_t* block_size, uint32_t* type_size);

/* Exact IEEE half -> single (dequant.cpp:222-248, fp16ToFloat).  Host function. */
float qvx_fp16_to_float(uint16_t h);

/* bfloat16 -> single: the 16 bits become the high half of the fp32 word (dequant.cpp:250-255,
 * bf16ToFloat; runtime/include/qorvix/runtime/dequant.hpp:51).  Host function. */
float qvx_bf16_to_float(uint16_t b);

/* ---- device entry points (device pointers, stream-ordered) --------------------------------- */

/* out[r] = dot(dequant(row r of W), x), r < rows.  Replaces qmatmul (qmatmul.cpp:28-62).
 * fp32 accumulation; within max|y-ref|/max|ref| <= 1e-3 of the exact sum.  The quantised-weight
 * kernels convert x per 64-element slot to 15-bit fixed point scaled by the slot's largest |x|, so an
 * element's conversion error is at most 3.1e-5 of that maximum (outlier channels of 1000x the typical
 * magnitude stay within the bar).  A non-finite activation makes its slot's step NaN: every output is
 * then NaN exactly where the reference's fp32 sum is non-finite (where the reference gives +-Inf, the
 * engine gives NaN). */
int qvx_qmatmul(float* d_out, const void* d_w, uint32_t type, const float* d_x, int rows, int cols,
                void* stream);

/* out[v * rows + r] for v < n_vec.  Replaces qmatmulN (qmatmul.cpp:64-115).  Each output is
 * bit-identical to qvx_qmatmul on that vector, as the reference promises (qmatmul.hpp:31-32).
 * Q4_K batches of 12 vectors or more on weights of >= 32 Mi elements, and of 24 or more on smaller
 * ones, on the one-vector kernel's shapes (cols a multiple of 256 up to 32768, aligned operands) run
 * on a many-vector form: the activations are converted once into a
 * stream-ordered temporary from the library's pool (nvec * cols * 2.25 bytes, plus 2 KiB per 32-row
 * tile and K range for batches up to 32 vectors), then the weights are streamed once per 64 vectors
 * (once per 16 up to 32 vectors) -- the reference's "dequantize each block once for all nVec dot
 * products" (qmatmul.hpp:24-32); smaller batches stream them once per 8 vectors and allocate
 * nothing, except on rows of >= 8192 elements from 5 to 23 vectors and on weights of <= 4 Mi elements
 * from 12 to 23, which stream them once per 16 on a split form whose K ranges are spread over
 * workgroups (a temporary of rows/32 * KQ * 1 or 2 KiB for the range partials; KQ = 4 or 16 ranges).
 * Q6_K batches of 3 vectors and of 5 or more, of 4 on weights of >= 8192 rows or columns and of 2
 * on weights of >= 65536 rows, with cols a multiple of 2048, stream the weights once per 16 vectors
 * (per 4 or 8 when the call has at most that many) on a matrix-core form whose K range is split over
 * workgroups by 2048-element blocks; for rows of more than one block it takes a stream-ordered
 * temporary for the block sums (rows/32 * blocks * 0.5, 1 or 2 KiB; without one the batch runs on
 * the VALU kernel, four vectors a launch) and adds them in a second launch.  A plan gives these calls
 * a workspace of its own, allocated by qvx_plan_instantiate, so its replays allocate nothing; on
 * shallow grids (<= 8 vectors, at most two 32-row tiles a workgroup) it also gives the call one
 * zeroed counter a 32-row tile, with which the kernel adds the block sums itself. */
int qvx_qmatmul_n(float* d_out, const void* d_w, uint32_t type, const float* d_X, int n_vec,
                  int rows, int cols, void* stream);

/* out[v * rows + r] = (W . X[v])[r] + bias[r] (d_bias [rows] fp32; NULL: no bias, exactly
 * qvx_qmatmul_n): the reference's wmatmulBias / wmatmulNBias (runtime/include/qorvix/runtime/
 * weights.hpp:58-80), the bias added after the product in fp32, so each output is the bit pattern of
 * qvx_qmatmul_n's output plus bias[r].  The arguments and checks of qvx_qmatmul_n.  The Q4_K batches
 * qvx_qmatmul_n runs on its many-vector form (above) add the bias in its epilogue; other
 * calls run the product, then one bias-add launch. */
int qvx_qmatmul_n_bias(float* d_out, const void* d_w, uint32_t type, const float* d_X, const float* d_bias,
                       int n_vec, int rows, int cols, void* stream);

/* Dequantise the first n / blockSize whole blocks of `type` to fp32, bit-exact with the reference's
 * dequantize (dequant.cpp:277-296) for every value but NaN payloads.  As there, n is not required
 * to be a whole number of blocks: the last n % blockSize outputs are left untouched. */
int qvx_dequantize(uint32_t type, const void* d_src, float* d_dst, size_t n, void* stream);

/* Dequantise row `row` (cols elements) of W.  Replaces dequantRow (qmatmul.cpp:117-126); as
 * there, the caller guarantees the row exists.  row < 0 -> QVX_E_RANGE. */
int qvx_dequant_row(const void* d_w, uint32_t type, int cols, int row, float* d_dst, void* stream);

/* ---- the decoder's ops on either side of the operator ----------------------------------- */
/* The reference's ops::rmsnorm (runtime/src/ops.cpp:8-13) on n_vec rows of n: out = x * scale * w,
 * scale = 1 / sqrt(sum x^2 / n + eps) formed in double.  The sum of squares is taken in the engine's
 * one canonical order (512-element chunks, 8-element runs, a fixed tree; the reference sums in
 * double element by element, so the scale may differ from it in the last bit), the order every
 * fused call below uses too, so normed inputs agree bit for bit across all routes.  n < 0 or
 * n > 16384 -> QVX_E_RANGE. */
int qvx_rmsnorm(float* d_out, const float* d_x, const float* d_w, float eps, int n_vec, int n, void* stream);
/* The reference's ops::swiglu (runtime/src/ops.cpp:96-100): out[i] = silu(gate[i]) * up[i],
 * silu(z) = z / (1 + exp(-z)), in fp32. */
int qvx_swiglu(float* d_out, const float* d_gate, const float* d_up, size_t n, void* stream);

/* Grouped GEMV: d_out[i] = W_i . xn for the n members (1 <= n <= QVX_GROUP_MAX, else QVX_E_NVEC),
 * each member's W_i of types[i] with rows[i] rows and the shared cols, xn = rmsnorm(x, d_norm_w,
 * eps) when d_norm_w is non-NULL, else x: the reference decoder's rmsnorm and the consecutive
 * wmatmuls of its output, the q / k / v projections (runtime/src/text_model.cpp:146-149), in one
 * call.  Each member's checks and outputs are qvx_qmatmul's, or qvx_qmatmul_n_rmsnorm's with a norm
 * (d_out[i] is bit-identical to that call on member i alone); a member with rows[i] <= 0 computes
 * nothing.  Up to 4 Q4_K members and one Q6_K member with aligned operands and cols a multiple of
 * 256 up to 16384 (of 512 with a norm) run as ONE launch (the dispatch ramp and drain paid once,
 * the norm folded into each workgroup's activation conversion); other groups run member by member. */
#define QVX_GROUP_MAX 8
int qvx_qmatmul_group(float* const* d_out, const void* const* d_w, const uint32_t* types, const int* rows, int n,
                      const float* d_x, const float* d_norm_w, float eps, int cols, void* stream);
/* y[v] = W . rmsnorm(x[v], norm_w, eps): the reference decoder's ops::rmsnorm followed by wmatmul
 * (runtime/src/text_model.cpp:146-149, 161-163, 171-172) in one call; the arguments and checks of
 * qvx_qmatmul_n plus d_norm_w [cols] (NULL -> QVX_E_NULL; cols > 16384 -> QVX_E_RANGE).  Where the GEMV kernel takes the shape
 * (Q4_K and the integer-dot formats, cols a multiple of 512 up to 16384, aligned operands) the norm
 * is folded into the kernel's activation conversion: one launch, no temporary; the per-vector
 * arithmetic does not depend on n_vec, so batches are bit-identical to single vectors.  Q6_K
 * batches the batched matrix-core form takes (cols a multiple of 2048; weights of >= 8192 rows or
 * columns, or 6 vectors or more) run the standalone norm into a stream-ordered temporary (n_vec *
 * cols * 4 bytes beside the form's block sums) and then that form: the norm forms the same bits as
 * the folded one, so these batches are bit-identical to single vectors too.  Otherwise a standalone
 * norm into a stream-ordered temporary, then qvx_qmatmul_n. */
int qvx_qmatmul_n_rmsnorm(float* d_out, const void* d_w, uint32_t type, const float* d_X,
                          const float* d_norm_w, float eps, int n_vec, int rows, int cols, void* stream);
/* out[v, i] = silu(g[v, i]) * u[v, i], g = W_gate . xn[v], u = W_up . xn[v], xn = rmsnorm(x[v])
 * when d_norm_w is non-NULL, else x[v]: the reference's gate / up wmatmuls and ops::swiglu
 * (text_model.cpp:161-165) in one call.  d_w_gu holds both weights interleaved in 16-row groups
 * (rows 32k .. 32k+15 = gate rows 16k .., rows 32k+16 .. 32k+31 = up rows 16k ..; build it with
 * qvx_interleave_rows16), 2 * ffn rows; out [n_vec, ffn].  ffn % 16 != 0 -> QVX_E_SHAPE.  Q4_K with
 * ffn % 16 == 0 and aligned operands runs fused (the gate and up tiles of a workgroup meet in its
 * epilogue); other calls run the product into a temporary and a standalone SwiGLU. */
int qvx_qmatmul_swiglu(float* d_out, const void* d_w_gu, uint32_t type, const float* d_X,
                       const float* d_norm_w, float eps, int n_vec, int ffn, int cols, void* stream);
/* Interleave two [rows, cols] weights of `type` in 16-row groups into d_dst (2 rows x cols), the
 * layout qvx_qmatmul_swiglu reads: a load-time repack of raw blocks (no reference counterpart;
 * the reference keeps gate and up apart, weights.hpp:22-97).  rows % 16 != 0 -> QVX_E_SHAPE. */
int qvx_interleave_rows16(void* d_dst, const void* d_a, const void* d_b, uint32_t type, int rows, int cols,
                          void* stream);

/* Prefill GEMM: out[m * rows + r] = sum_k X[m, k] * dequant(W)[r, k] for m < M, X fp16 [M, cols].
 * No reference counterpart (the reference prefills token by token); semantics are qmatmulN's
 * with X converted fp16 -> fp32 exactly.  variant = QVX_GEMM_BF16 | QVX_GEMM_F16 | QVX_GEMM_I8;
 * tolerance 2e-2 max-relative against the exact sum.  type: every type qvx_qmatmul takes, each on the
 * engine's own matrix-core kernels (no library GEMM), each weight element rounded to fp16 / bf16
 * from its exact dequantised value.  Q4_K runs on raw-block MFMA kernels; Q6_K with X 16-byte and W
 * 4-byte aligned on its own raw-block MFMA kernels (cols a multiple of 512: the Q4_K kernels'
 * pipeline, blocks dequantised in registers; else cols a multiple of 64: a dequantising kernel),
 * except from M = 1024 on a weight of >= 32 Mi elements, where the 16-bit route below is faster.
 * Other types, and Q6_K calls those kernels decline, are dequantised into a stream-ordered 16-bit
 * temporary (fp16, bf16 for QVX_GEMM_BF16; per panel of rows) and multiplied by the plain 16-bit MFMA
 * GEMM of qvx_gemm16.  QVX_GEMM_I8 takes Q4_K only (other types: QVX_E_TYPE).  Grids smaller than
 * the chip (small M) split K across workgroups; the last split of each output tile adds the partial
 * tiles in split order, so every call returns the same bits for the same inputs. */
int qvx_qgemm_f16(float* d_out, const void* d_w, uint32_t type, const uint16_t* d_X, int M,
                  int rows, int cols, int variant, void* stream);

/* The prefill GEMM without any device allocation: the arguments, checks, kernels and results of
 * qvx_qgemm_f16, for callers that cannot allocate (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  No reference counterpart.  One exception: the large Q6_K calls
 * qvx_qgemm_f16 runs through a 16-bit weight (M >= 1024, >= 32 Mi weight elements) stay on the
 * raw-block kernel here, whose results agree with those within the GEMM tolerance, not bit for bit.  Its temporaries (the bf16 or Q8 copy
 * of X, a K split's partial tiles, and for the types without a raw-block kernel the 16-bit weight)
 * live in one fixed scratch array per device, of QVX_NOALLOC_SCRATCH_BYTES, held from the first call
 * on a device until the process ends; no call makes hipMalloc, hipFree or an allocating library
 * call.  A call whose temporaries exceed the scratch -> QVX_E_RANGE (QVX_GEMM_BF16 needs 2*M*cols
 * bytes, QVX_GEMM_I8 about 1.25*M*cols, QVX_GEMM_F16 none; plus, when a grid smaller than the chip
 * splits K, 128 KiB of partial tile per tile and split -- qvx_qgemm_plan_q4k reports both for Q4_K;
 * the types dequantised to 16 bits run panel by panel of at least 256 weight rows, each panel's
 * 16-bit weight (2*256*cols bytes at the least) sharing the scratch with the copy of X).  Every call
 * on a device shares that device's scratch: calls that overlap on one device (different streams, or
 * host threads) race and must be ordered by the caller. */
#define QVX_NOALLOC_SCRATCH_BYTES (64u << 20)
int qvx_qgemm_f16_noalloc(float* d_out, const void* d_w, uint32_t type, const uint16_t* d_X, int M,
                          int rows, int cols, int variant, void* stream);

/* Tile plan of the Q4_K bf16 / fp16 GEMM kernels behind qvx_qgemm_f16 for an M x rows x cols call
 * on a device with `cus` compute units (cus <= 0: the current device's).  No reference
 * counterpart: a host-only query for tests and for callers sizing concurrent work.  Writes up to
 * `cap` launches of 8 ints each -- tile tokens BM, K splits, tiles, cols_a, mt_a, base_a, mt_b,
 * base_b: weight-row columns 0..cols_a-1 (256 rows each) hold mt_a tiles of BM tokens from token
 * base_a, the remaining columns mt_b tiles from token base_b -- and returns the number of launches
 * (1 or 2), or QVX_E_SHAPE when M, rows or cols is not positive or cols % 256 != 0. */
int qvx_qgemm_plan_q4k(int M, int rows, int cols, int cus, int* desc, int cap);

/* Plain 16-bit GEMM on the matrix cores: out[m * N + n] = sum_k X[m, k] * B[n, k], X [M, K] and
 * B [N, K] row-major bf16 (variant QVX_GEMM_BF16) or fp16 (QVX_GEMM_F16) bits, fp32 accumulation
 * and output.  No reference counterpart: the GEMM behind qvx_qgemm_f16 for weights dequantised to
 * 16 bits (qvx_dequantize16), for callers that keep a dequantised copy of a weight and multiply it
 * many times.  The kernel takes K in multiples of 64 and 16-byte-aligned operands; other calls run
 * on zero-padded copies from the library's stream-ordered pool, as do the partial tiles of a K split
 * (grids smaller than the chip; the partials are added in split order, so results do not vary
 * between runs).  M, N or K < 0 -> QVX_E_SHAPE; M or N == 0 is a no-op; K == 0 writes zeros. */
int qvx_gemm16(float* d_out, const uint16_t* d_X, const uint16_t* d_B, int M, int N, int K, int variant,
               void* stream);

/* Dequantise the first n / blockSize whole blocks of `type` to 16 bits: the reference's dequantised
 * value (dequant.cpp:277-296) rounded once to nearest-even bf16 (bf16 != 0) or fp16 -- the weight
 * operand of the prefill GEMM.  No reference counterpart. */
int qvx_dequantize16(uint32_t type, const void* d_src, uint16_t* d_dst, size_t n, int bf16, void* stream);

/* Per-32 Q8 activation quantiser used by QVX_GEMM_I8 (no reference counterpart): for row m and
 * block j, scale = amax/127, q = round-half-away(x * 127/amax) clamped to +-127, qsum = sum q.
 * d_q int8 [M, K], d_scale fp32 [M, K/32], d_qsum int32 [M, K/32]; K % 32 == 0. */
int qvx_quantize_act_q8(const uint16_t* d_X, int M, int K, int8_t* d_q, float* d_scale,
                        int32_t* d_qsum, void* stream);

/* Fill a [rows, cols] weight of `type` with seeded synthetic blocks on the device (benchmark and
 * test data; no reference counterpart), for Q8_0, Q4_0, Q4_K, Q5_K and Q6_K.  Scales are
 * fp16(|N(0,1)| * scale_mul) (Q4_K / Q5_K: d and dmin;
 * Q6_K: d), quant bytes uniform, Q6_K int8 sub-scales uniform over [-128, 127].  Deterministic in
 * (seed, byte position). */
int qvx_fill_synthetic(void* d_w, uint32_t type, int rows, int cols, uint64_t seed, float scale_mul,
                       void* stream);

/* Fill n fp32 values with N(0,1) * mul (seeded, deterministic), or n fp16 values. */
int qvx_fill_normal_f32(float* d_x, size_t n, uint64_t seed, float mul, void* stream);
int qvx_fill_normal_f16(uint16_t* d_x, size_t n, uint64_t seed, float mul, void* stream);

/* Bare streaming read of n bytes (benchmark only, no reference counterpart): the HBM read rate a
 * single launch reaches, beside which the GEMV's rate is judged.  One 16-byte load per thread; *d_flag
 * is written (1) only if a 16-byte word of the data equals the fixed pattern 0x5A17C0DE x 4, so for
 * other data nothing is stored.  n % 16 == 0 and d_src 16-byte aligned, else QVX_E_RANGE. */
int qvx_bench_read(const void* d_src, size_t n, uint32_t* d_flag, void* stream);

/* ---- plans: a recorded sequence of GEMV calls replayed as one HIP graph ------------------- */
/* The form in which the reference's CUDA backend runs a decode step: the same type-switched
 * matmul launches (cuda/src/cuda_backend.cu:1523-1542, matmul / matmulS) issued on one stream and
 * captured into a graph, so a token's projections replay with one launch.  A plan holds device
 * pointers only; the buffers must outlive it.  Plans are not thread-safe; distinct plans are. */
typedef struct qvx_plan qvx_plan;
/* New empty plan bound to the current device. */
int qvx_plan_create(qvx_plan** plan);
/* Append out = W X (the arguments and checks of qvx_qmatmul_n; nothing runs).  A call with
 * rows <= 0 is accepted and records nothing.  Appending to an instantiated plan -> QVX_E_STATE. */
int qvx_plan_add_qmatmul_n(qvx_plan* plan, float* d_out, const void* d_w, uint32_t type,
                           const float* d_X, int n_vec, int rows, int cols);
/* Record a qvx_qmatmul_group call (the same arguments and checks; with a norm, every member must be
 * one a kernel folds the norm into, as for qvx_plan_add_qmatmul_n_rmsnorm, else QVX_E_SHAPE). */
int qvx_plan_add_qmatmul_group(qvx_plan* plan, float* const* d_out, const void* const* d_w, const uint32_t* types,
                               const int* rows, int n, const float* d_x, const float* d_norm_w, float eps,
                               int cols);
/* Append a fused call (the arguments and checks of qvx_qmatmul_n_rmsnorm / qvx_qmatmul_swiglu).  A
 * replay allocates nothing, so only calls a kernel folds the norm / SwiGLU into, or whose norm the
 * plan's workspace holds (the Q6_K batches above), are accepted (others -> QVX_E_SHAPE). */
int qvx_plan_add_qmatmul_n_rmsnorm(qvx_plan* plan, float* d_out, const void* d_w, uint32_t type,
                                   const float* d_X, const float* d_norm_w, float eps, int n_vec,
                                   int rows, int cols);
int qvx_plan_add_qmatmul_swiglu(qvx_plan* plan, float* d_out, const void* d_w_gu, uint32_t type,
                                const float* d_X, const float* d_norm_w, float eps, int n_vec,
                                int ffn, int cols);
/* Calls added between qvx_plan_fork and qvx_plan_join are independent of each other (the graph
 * gets one branch per call, so their kernels may overlap on the device); all of them follow every
 * call before the fork and precede every call after the join -- as the decoder's q/k/v
 * projections all read the normed state (text_model.cpp:147-150).  Forking twice, or joining
 * without a fork, -> QVX_E_STATE. */
int qvx_plan_fork(qvx_plan* plan);
int qvx_plan_join(qvx_plan* plan);
/* Number of recorded calls. */
int qvx_plan_size(const qvx_plan* plan);
/* Capture the recorded calls into a HIP graph on the plan's device and instantiate it (an open
 * fork is joined first).  Allocates the device workspace of the plan's many-vector calls (one slice
 * shared by the calls in order, disjoint slices for the calls of one fork), freed with the plan. */
int qvx_plan_instantiate(qvx_plan* plan);
/* Replay the graph on `stream` (stream-ordered, asynchronous).  Not instantiated -> QVX_E_STATE. */
int qvx_plan_launch(qvx_plan* plan, void* stream);
/* Issue the recorded calls one by one on `stream` (no graph): the same kernels and arguments once
 * the plan is instantiated; before that a many-vector call, having no workspace yet, takes the
 * chunked batched form (the same output bits). */
int qvx_plan_run_eager(const qvx_plan* plan, void* stream);
/* Free the plan and its graph (NULL is a no-op). */
void qvx_plan_destroy(qvx_plan* plan);
/* ---- GGUF files: parse, locate tensors, upload ------------------------------------------- */
/* GGUF files, in place of the reference's GgufFile (gguf/include/qorvix/gguf/gguf_file.hpp:47-105):
 * a reader of the public GGUF container, versions 1-3, little-endian.  Malformed data returns
 * QVX_E_FORMAT and keeps a message for qvx_gguf_last_error (per thread); a file is refused when a
 * read would pass its end, a value type is not one of the format's 13, a tensor has more than 4
 * dimensions, a block-quantised tensor's rows are not whole blocks, a tensor offset is not a
 * multiple of the alignment (general.alignment, a u32 power of two, default 32), a key or tensor
 * name appears twice, sizes overflow 64 bits, or a tensor's bytes lie outside the data section.
 * Arrays of arrays parse (the format allows them) but their elements are not exposed.  Nothing is
 * copied: the handle indexes the mapping (qvx_gguf_open) or the caller's buffer (qvx_gguf_parse),
 * and values are decoded when asked for.  Tensor dimensions are in ggml order (dims[0] is the row
 * length, `cols`; dims[1] the row count, `rows`); offsets are relative to the data section
 * (qvx_gguf_data_offset); n_bytes is the on-disk size from the type's block traits, 0 for a type id
 * without traits. */
typedef struct qvx_gguf qvx_gguf;
/* Memory-map `path` read-only and parse it (GgufFile::open, gguf_file.hpp:54-55). */
int qvx_gguf_open(const char* path, qvx_gguf** out);
/* Parse a caller's buffer, which must outlive the handle (GgufFile::parse, gguf_file.hpp:51-52). */
int qvx_gguf_parse(const void* data, size_t size, qvx_gguf** out);
void qvx_gguf_close(qvx_gguf* f);
/* Message of the last failed open / parse on this thread ("" after a success). */
const char* qvx_gguf_last_error(void);
uint32_t qvx_gguf_version(const qvx_gguf* f);
uint32_t qvx_gguf_alignment(const qvx_gguf* f);   /* general.alignment, default 32 */
uint64_t qvx_gguf_data_offset(const qvx_gguf* f); /* dataOffset(), gguf_file.hpp:62 */
int64_t qvx_gguf_tensor_count(const qvx_gguf* f);
int64_t qvx_gguf_meta_count(const qvx_gguf* f);
/* Index of the tensor named `name`, -1 if absent (tensor(), gguf_file.hpp:65). */
int64_t qvx_gguf_find_tensor(const qvx_gguf* f, const char* name);
/* Tensor i (GgufTensor, gguf_file.hpp:27-35): any output may be NULL; dims receives 8 values
 * (zeros past n_dims, which is at most 4).  i out of range -> QVX_E_RANGE. */
int qvx_gguf_tensor_info(const qvx_gguf* f, int64_t i, const char** name, uint32_t* type, uint32_t* n_dims,
                         uint64_t* dims, uint64_t* offset, uint64_t* n_elements, uint64_t* n_bytes);
/* Host address of tensor i's bytes in the mapping / buffer, NULL when it does not carry them. */
const void* qvx_gguf_tensor_data(const qvx_gguf* f, int64_t i);
/* Copy tensor i's raw blocks to device memory (stream-ordered; the GPU weight upload of
 * cuda_backend.cu:1300-1309 with weightBytes, :1246-1255).  dst_bytes < n_bytes -> QVX_E_RANGE;
 * a type without traits -> QVX_E_TYPE.  The GEMV / GEMM entry points take the blocks as they are. */
int qvx_gguf_upload(const qvx_gguf* f, int64_t i, void* d_dst, size_t dst_bytes, void* stream);
/* Metadata key i in file order, NULL past the end (metadata(), gguf_file.hpp:68-70). */
const char* qvx_gguf_meta_key(const qvx_gguf* f, int64_t i);
/* Value type tag of `key` (0..12 as on disk), its element type for an array (else the same tag),
 * and its element count (1 for a scalar).  Absent -> QVX_E_RANGE. */
int qvx_gguf_meta_type(const qvx_gguf* f, const char* key, uint32_t* type, uint32_t* elem_type, uint64_t* count);
/* Element `index` of `key` (0 for a scalar), in the categories of the reference's getU64 / getF64 /
 * getBool / getString (gguf_file.hpp:74-78): integers and bools as u64 / i64, numbers other than
 * bools as f64.  Absent or index past the end -> QVX_E_RANGE; wrong category (or an element of an
 * array of arrays) -> QVX_E_TYPE.  A string points into the file and is not NUL-terminated; *len
 * holds its length. */
int qvx_gguf_meta_u64(const qvx_gguf* f, const char* key, uint64_t index, uint64_t* out);
int qvx_gguf_meta_i64(const qvx_gguf* f, const char* key, uint64_t index, int64_t* out);
int qvx_gguf_meta_f64(const qvx_gguf* f, const char* key, uint64_t index, double* out);
int qvx_gguf_meta_bool(const qvx_gguf* f, const char* key, uint64_t index, int* out);
int qvx_gguf_meta_string(const qvx_gguf* f, const char* key, uint64_t index, const char** out, size_t* len);
/* ---- host entry points (host pointers, synchronous) --------------------------------------- */
/* The reference's CPU signatures (qmatmul.hpp:14-36, dequant.hpp:12-21) over the GPU kernels:
 * weight, x and out live in host memory; the call uploads, computes on the current device and
 * downloads before returning. */
int qvx_qmatmul_host(float* out, const void* w, uint32_t type, const float* x, int rows, int cols);
int qvx_qmatmul_n_host(float* out, const void* w, uint32_t type, const float* X, int n_vec, int rows,
                       int cols);
int qvx_dequantize_host(uint32_t type, const void* src, float* dst, size_t n);
int qvx_dequant_row_host(const void* w, uint32_t type, int cols, int row, float* dst);

#ifdef __cplusplus
}
#endif

#endif /* QVX_H */
