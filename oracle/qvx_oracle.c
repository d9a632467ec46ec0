/*
 * qvx_oracle.c -- CPU restatement of the QorVix quantized-matmul path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker for the HIP engine under
 * qorvix_amd/: only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg may load it, and only to check or to time beside the GPU.  The product
 * never calls it.
 *
 * What it restates (behaviour, not text), with the reference file:line each
 * function follows:
 *   qvxo_fp16_to_float    runtime/src/dequant.cpp:222-248  (exact IEEE half->single,
 *                         subnormals normalised, Inf/NaN keep their payload)
 *   qvxo_bf16_to_float    runtime/src/dequant.cpp:250-255
 *   qvxo_type_traits      gguf/src/gguf_types.cpp:15-54    (ggml type id -> block size / bytes)
 *   qvxo_can_dequantize   runtime/src/dequant.cpp:257-275
 *   qvxo_dequantize       runtime/src/dequant.cpp:38-210,277-296 (serial per-block formulas)
 *   qvxo_dot_f32          runtime/src/cpu_features.cpp:34-75,129-151 (avx512 > avx2+fma > scalar)
 *   qvxo_qmatmul          runtime/src/qmatmul.cpp:28-62    (256-element chunks, OpenMP static rows)
 *   qvxo_qmatmul_n        runtime/src/qmatmul.cpp:64-115   (row dequantised once, vectors tiled by 64)
 *   qvxo_dequant_row      runtime/src/qmatmul.cpp:117-126
 *   qvxo_supports         runtime/src/qmatmul.cpp:24-26
 *   qvxo_rmsnorm          runtime/src/ops.cpp:8-13         (sum of squares in double, scale in
 *                         float, out = x * scale * w)
 *   qvxo_swiglu           runtime/src/ops.cpp:96-100       (silu(g) * u, silu(z) = z / (1 + exp(-z)))
 * and the build-defined parts that have no reference counterpart:
 *   qvxo_matmul_f64       exact dequant values x f32 activations, summed in double
 *                         (the tolerance oracle for every GEMV/GEMM)
 *   qvxo_quantize_q8_act  per-32 Q8 activation quantiser for the int8 MFMA GEMM
 *                         (scale = amax/127 in fp32, q = round-half-away(x/scale))
 *
 * Parity pins (each checked in tests/test_oracle.py):
 *   - dequant: known-answer cases of tests/dequant_test.cpp:24-135, closed-form
 *     RN(exact formula) computed in integers/double for every type, and bit-identity
 *     with oracle/_ref (the reference's own dequant.cpp built from its sources);
 *   - qmatmul / qmatmulN / dequantRow: tests/qmatmul_test.cpp:41-168 cases, the CUDA
 *     self-test patterns (cuda/src/cuda_backend.cu:551-573,721-748,793-825) against
 *     their double references, bit-identity batched vs unbatched, and bit-identity with
 *     oracle/_ref on random blocks;
 *   - fp16 decode: all 65536 encodings against numpy's float16;
 *   - qvxo_matmul_f64: brute-force Fraction sums on tiny inputs;
 *   - rmsnorm / swiglu: bit-identity with oracle/_ref (the reference's own ops.cpp built from
 *     its sources), and what the mathematics fixes: the output's mean square is 1 for eps = 0 and
 *     unit weights, rmsnorm is invariant under x -> a x, silu(0) = 0 and silu(z) -> z, 0 at the
 *     tails, swiglu is linear in up.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#if defined(__x86_64__) && (defined(__GNUC__) || defined(__clang__))
#define QVXO_X86 1
#include <immintrin.h>
#endif

#define QVXO_EXPORT __attribute__((visibility("default")))

/* ---- fp16 / bf16 --------------------------------------------------------------------------- */

QVXO_EXPORT float qvxo_fp16_to_float(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t e = (h >> 10) & 0x1Fu;
  uint32_t m = h & 0x3FFu;
  uint32_t bits;
  if (e == 0) {
    if (m == 0) {
      bits = sign;
    } else {
      /* subnormal half: shift the mantissa up until its leading one reaches bit 10 */
      uint32_t fe = 113; /* 127 - 15 + 1 */
      while (!(m & 0x400u)) {
        m <<= 1;
        fe--;
      }
      bits = sign | (fe << 23) | ((m & 0x3FFu) << 13);
    }
  } else if (e == 31) {
    bits = sign | 0x7F800000u | (m << 13);
  } else {
    bits = sign | ((e + 112u) << 23) | (m << 13);
  }
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

QVXO_EXPORT float qvxo_bf16_to_float(uint16_t b) {
  uint32_t bits = (uint32_t)b << 16;
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

static inline uint16_t rd16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* ---- ggml type traits ------------------------------------------------------------------------ */

typedef struct {
  uint32_t id;
  uint32_t block;
  uint32_t bytes;
} qvxo_traits;

/* On-disk ggml ids with (elements per block, bytes per block); the public ggml block structs. */
static const qvxo_traits k_types[] = {
    {0, 1, 4},     {1, 1, 2},     {2, 32, 18},   {3, 32, 20},   {6, 32, 22},   {7, 32, 24},
    {8, 32, 34},   {9, 32, 36},   {10, 256, 84}, {11, 256, 110}, {12, 256, 144}, {13, 256, 176},
    {14, 256, 210}, {15, 256, 292}, {16, 256, 66}, {17, 256, 74}, {18, 256, 98},  {19, 256, 50},
    {20, 32, 18},  {21, 256, 110}, {22, 256, 82}, {23, 256, 136}, {24, 1, 1},     {25, 1, 2},
    {26, 1, 4},    {27, 1, 8},     {28, 1, 8},    {29, 256, 56},  {30, 1, 2},
};

static const qvxo_traits* traits_of(uint32_t t) {
  for (size_t i = 0; i < sizeof(k_types) / sizeof(k_types[0]); ++i)
    if (k_types[i].id == t) return &k_types[i];
  return NULL;
}

/* Returns 1 and fills block/bytes for a known id, 0 otherwise. */
QVXO_EXPORT int qvxo_type_traits(uint32_t t, uint32_t* block, uint32_t* bytes) {
  const qvxo_traits* tr = traits_of(t);
  if (!tr) return 0;
  if (block) *block = tr->block;
  if (bytes) *bytes = tr->bytes;
  return 1;
}

QVXO_EXPORT int qvxo_can_dequantize(uint32_t t) {
  switch (t) {
    case 0: case 1: case 30: case 8: case 9: case 2: case 3: case 6: case 7: case 12: case 13:
    case 14:
      return 1;
    default:
      return 0;
  }
}

/* ---- per-type dequantisers (serial; one call covers n/block whole blocks) ------------------ */

static void dq_q8_0(const uint8_t* s, float* y, size_t n) {
  for (size_t b = 0; b < n / 32; ++b, s += 34, y += 32) {
    const float d = qvxo_fp16_to_float(rd16(s));
    for (int i = 0; i < 32; ++i) y[i] = d * (float)(int8_t)s[2 + i];
  }
}

static void dq_q8_1(const uint8_t* s, float* y, size_t n) {
  for (size_t b = 0; b < n / 32; ++b, s += 36, y += 32) {
    const float d = qvxo_fp16_to_float(rd16(s));
    for (int i = 0; i < 32; ++i) y[i] = d * (float)(int8_t)s[4 + i];
  }
}

static void dq_q4_0(const uint8_t* s, float* y, size_t n) {
  for (size_t b = 0; b < n / 32; ++b, s += 18, y += 32) {
    const float d = qvxo_fp16_to_float(rd16(s));
    for (int i = 0; i < 16; ++i) {
      y[i] = (float)((s[2 + i] & 15) - 8) * d;
      y[i + 16] = (float)((s[2 + i] >> 4) - 8) * d;
    }
  }
}

static void dq_q4_1(const uint8_t* s, float* y, size_t n) {
  for (size_t b = 0; b < n / 32; ++b, s += 20, y += 32) {
    const float d = qvxo_fp16_to_float(rd16(s));
    const float m = qvxo_fp16_to_float(rd16(s + 2));
    for (int i = 0; i < 16; ++i) {
      y[i] = (float)(s[4 + i] & 15) * d + m;
      y[i + 16] = (float)(s[4 + i] >> 4) * d + m;
    }
  }
}

static void dq_q5_0(const uint8_t* s, float* y, size_t n) {
  for (size_t b = 0; b < n / 32; ++b, s += 22, y += 32) {
    const float d = qvxo_fp16_to_float(rd16(s));
    uint32_t qh;
    memcpy(&qh, s + 2, 4);
    for (int i = 0; i < 16; ++i) {
      const int lo = (s[6 + i] & 15) | (int)(((qh >> i) & 1u) << 4);
      const int hi = (s[6 + i] >> 4) | (int)(((qh >> (i + 16)) & 1u) << 4);
      y[i] = (float)(lo - 16) * d;
      y[i + 16] = (float)(hi - 16) * d;
    }
  }
}

static void dq_q5_1(const uint8_t* s, float* y, size_t n) {
  for (size_t b = 0; b < n / 32; ++b, s += 24, y += 32) {
    const float d = qvxo_fp16_to_float(rd16(s));
    const float m = qvxo_fp16_to_float(rd16(s + 2));
    uint32_t qh;
    memcpy(&qh, s + 4, 4);
    for (int i = 0; i < 16; ++i) {
      const int lo = (s[8 + i] & 15) | (int)(((qh >> i) & 1u) << 4);
      const int hi = (s[8 + i] >> 4) | (int)(((qh >> (i + 16)) & 1u) << 4);
      y[i] = (float)lo * d + m;
      y[i + 16] = (float)hi * d + m;
    }
  }
}

/* 6-bit (scale, min) of sub-block j from the 12 packed K-quant scale bytes (public ggml layout). */
QVXO_EXPORT void qvxo_k4_scale_min(int j, const uint8_t* q, uint8_t* sc, uint8_t* mn) {
  if (j < 4) {
    *sc = q[j] & 63;
    *mn = q[j + 4] & 63;
  } else {
    *sc = (uint8_t)((q[j + 4] & 15) | ((q[j - 4] >> 6) << 4));
    *mn = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
  }
}

static void dq_q4_k(const uint8_t* s, float* y, size_t n) {
  for (size_t b = 0; b < n / 256; ++b, s += 144) {
    const float d = qvxo_fp16_to_float(rd16(s));
    const float dmin = qvxo_fp16_to_float(rd16(s + 2));
    const uint8_t* q = s + 16;
    for (int c = 0; c < 4; ++c, q += 32) {
      uint8_t sc0, m0, sc1, m1;
      qvxo_k4_scale_min(2 * c, s + 4, &sc0, &m0);
      qvxo_k4_scale_min(2 * c + 1, s + 4, &sc1, &m1);
      const float ds0 = d * (float)sc0, dm0 = dmin * (float)m0;
      const float ds1 = d * (float)sc1, dm1 = dmin * (float)m1;
      for (int l = 0; l < 32; ++l) *y++ = ds0 * (float)(q[l] & 15) - dm0;
      for (int l = 0; l < 32; ++l) *y++ = ds1 * (float)(q[l] >> 4) - dm1;
    }
  }
}

static void dq_q5_k(const uint8_t* s, float* y, size_t n) {
  for (size_t b = 0; b < n / 256; ++b, s += 176) {
    const float d = qvxo_fp16_to_float(rd16(s));
    const float dmin = qvxo_fp16_to_float(rd16(s + 2));
    const uint8_t* qh = s + 16;
    const uint8_t* ql = s + 48;
    for (int c = 0; c < 4; ++c, ql += 32) {
      uint8_t sc0, m0, sc1, m1;
      qvxo_k4_scale_min(2 * c, s + 4, &sc0, &m0);
      qvxo_k4_scale_min(2 * c + 1, s + 4, &sc1, &m1);
      const float ds0 = d * (float)sc0, dm0 = dmin * (float)m0;
      const float ds1 = d * (float)sc1, dm1 = dmin * (float)m1;
      const uint8_t b0 = (uint8_t)(1u << (2 * c)), b1 = (uint8_t)(2u << (2 * c));
      for (int l = 0; l < 32; ++l) *y++ = ds0 * (float)((ql[l] & 15) + ((qh[l] & b0) ? 16 : 0)) - dm0;
      for (int l = 0; l < 32; ++l) *y++ = ds1 * (float)((ql[l] >> 4) + ((qh[l] & b1) ? 16 : 0)) - dm1;
    }
  }
}

static void dq_q6_k(const uint8_t* s, float* y, size_t n) {
  for (size_t b = 0; b < n / 256; ++b, s += 210) {
    const float d = qvxo_fp16_to_float(rd16(s + 208));
    for (int h = 0; h < 2; ++h) {
      const uint8_t* ql = s + 64 * h;
      const uint8_t* qh = s + 128 + 32 * h;
      const int8_t* sc = (const int8_t*)(s + 192 + 8 * h);
      float* o = y + 256 * b + 128 * h;
      for (int l = 0; l < 32; ++l) {
        const int t = l / 16;
        const int q0 = ((ql[l] & 15) | (((qh[l] >> 0) & 3) << 4)) - 32;
        const int q1 = ((ql[l + 32] & 15) | (((qh[l] >> 2) & 3) << 4)) - 32;
        const int q2 = ((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
        const int q3 = ((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
        o[l] = d * (float)sc[t] * (float)q0;
        o[l + 32] = d * (float)sc[t + 2] * (float)q1;
        o[l + 64] = d * (float)sc[t + 4] * (float)q2;
        o[l + 96] = d * (float)sc[t + 6] * (float)q3;
      }
    }
  }
}

QVXO_EXPORT int qvxo_dequantize(uint32_t t, const void* src, float* dst, size_t n) {
  const uint8_t* s = (const uint8_t*)src;
  switch (t) {
    case 0: memcpy(dst, src, n * sizeof(float)); return 1;
    case 1: for (size_t i = 0; i < n; ++i) dst[i] = qvxo_fp16_to_float(rd16(s + 2 * i)); return 1;
    case 30: for (size_t i = 0; i < n; ++i) dst[i] = qvxo_bf16_to_float(rd16(s + 2 * i)); return 1;
    case 8: dq_q8_0(s, dst, n); return 1;
    case 9: dq_q8_1(s, dst, n); return 1;
    case 2: dq_q4_0(s, dst, n); return 1;
    case 3: dq_q4_1(s, dst, n); return 1;
    case 6: dq_q5_0(s, dst, n); return 1;
    case 7: dq_q5_1(s, dst, n); return 1;
    case 12: dq_q4_k(s, dst, n); return 1;
    case 13: dq_q5_k(s, dst, n); return 1;
    case 14: dq_q6_k(s, dst, n); return 1;
    default: return 0;
  }
}

/* ---- fp32 dot with runtime SIMD dispatch ---------------------------------------------------- */

typedef float (*dot_fn)(const float*, const float*, int);

static float dot_scalar(const float* a, const float* b, int n) {
  float r = 0.0f;
  for (int i = 0; i < n; ++i) r += a[i] * b[i];
  return r;
}

#if defined(QVXO_X86)
/* Two 8-wide FMA accumulators over 16-element steps, an 8-wide tail, horizontal sum, scalar tail. */
__attribute__((target("avx2,fma"))) static float dot_avx2(const float* a, const float* b, int n) {
  __m256 acc0 = _mm256_setzero_ps(), acc1 = _mm256_setzero_ps();
  int i = 0;
  for (; i + 16 <= n; i += 16) {
    acc0 = _mm256_fmadd_ps(_mm256_loadu_ps(a + i), _mm256_loadu_ps(b + i), acc0);
    acc1 = _mm256_fmadd_ps(_mm256_loadu_ps(a + i + 8), _mm256_loadu_ps(b + i + 8), acc1);
  }
  for (; i + 8 <= n; i += 8) acc0 = _mm256_fmadd_ps(_mm256_loadu_ps(a + i), _mm256_loadu_ps(b + i), acc0);
  acc0 = _mm256_add_ps(acc0, acc1);
  float lanes[8];
  _mm256_storeu_ps(lanes, acc0);
  float r = lanes[0] + lanes[1] + lanes[2] + lanes[3] + lanes[4] + lanes[5] + lanes[6] + lanes[7];
  for (; i < n; ++i) r += a[i] * b[i];
  return r;
}

/* One 16-wide FMA accumulator, the compiler's 512-bit horizontal add, scalar tail. */
__attribute__((target("avx512f"))) static float dot_avx512(const float* a, const float* b, int n) {
  __m512 acc = _mm512_setzero_ps();
  int i = 0;
  for (; i + 16 <= n; i += 16) acc = _mm512_fmadd_ps(_mm512_loadu_ps(a + i), _mm512_loadu_ps(b + i), acc);
  float r = _mm512_reduce_add_ps(acc);
  for (; i < n; ++i) r += a[i] * b[i];
  return r;
}
#endif

static dot_fn g_dot = 0;
static const char* g_dot_name = "scalar";

static void pick_dot(void) {
  if (g_dot) return;
  dot_fn f = dot_scalar;
  const char* name = "scalar";
#if defined(QVXO_X86)
  __builtin_cpu_init();
  if (__builtin_cpu_supports("avx512f")) {
    f = dot_avx512;
    name = "avx512";
  } else if (__builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma")) {
    f = dot_avx2;
    name = "avx2";
  }
#endif
  g_dot_name = name;
  g_dot = f;
}

__attribute__((constructor)) static void qvxo_init(void) { pick_dot(); }

QVXO_EXPORT const char* qvxo_dot_kernel(void) {
  pick_dot();
  return g_dot_name;
}

QVXO_EXPORT float qvxo_dot_f32(const float* a, const float* b, int n) {
  pick_dot();
  return g_dot(a, b, n);
}

/* ---- the operator -------------------------------------------------------------------------- */

enum { K_MAX_BLOCK = 256, K_VEC_TILE = 64 };

QVXO_EXPORT int qvxo_supports(uint32_t t) { return qvxo_can_dequantize(t) && traits_of(t) != NULL; }

QVXO_EXPORT int qvxo_qmatmul(float* out, const void* weight, uint32_t t, const float* x, int rows,
                             int cols) {
  const qvxo_traits* tr = traits_of(t);
  if (!tr || !qvxo_can_dequantize(t)) return 0;
  const int bs = (int)tr->block;
  if (bs <= 0 || bs > K_MAX_BLOCK || cols % bs != 0) return 0;
  const size_t row_bytes = (size_t)(cols / bs) * tr->bytes;
  const int per_batch = (K_MAX_BLOCK / bs) * bs; /* whole blocks filling at most 256 floats */
  const uint8_t* base = (const uint8_t*)weight;
  pick_dot();
#pragma omp parallel for schedule(static)
  for (int r = 0; r < rows; ++r) {
    const uint8_t* rp = base + (size_t)r * row_bytes;
    float buf[K_MAX_BLOCK];
    float acc = 0.0f;
    for (int e = 0; e < cols; e += per_batch) {
      const int n = cols - e < per_batch ? cols - e : per_batch;
      qvxo_dequantize(t, rp + (size_t)(e / bs) * tr->bytes, buf, (size_t)n);
      acc += g_dot(buf, x + e, n);
    }
    out[r] = acc;
  }
  return 1;
}

QVXO_EXPORT int qvxo_qmatmul_n(float* out, const void* weight, uint32_t t, const float* X, int nvec,
                               int rows, int cols) {
  if (nvec <= 0) return 0;
  if (nvec == 1) return qvxo_qmatmul(out, weight, t, X, rows, cols);
  const qvxo_traits* tr = traits_of(t);
  if (!tr || !qvxo_can_dequantize(t)) return 0;
  const int bs = (int)tr->block;
  if (bs <= 0 || bs > K_MAX_BLOCK || cols % bs != 0) return 0;
  const size_t row_bytes = (size_t)(cols / bs) * tr->bytes;
  const int per_batch = (K_MAX_BLOCK / bs) * bs;
  const uint8_t* base = (const uint8_t*)weight;
  pick_dot();
#pragma omp parallel
  {
    float* row = (float*)malloc(sizeof(float) * (size_t)(cols > 0 ? cols : 1));
#pragma omp for schedule(static)
    for (int r = 0; r < rows; ++r) {
      const uint8_t* rp = base + (size_t)r * row_bytes;
      for (int e = 0; e < cols; e += per_batch) {
        const int n = cols - e < per_batch ? cols - e : per_batch;
        qvxo_dequantize(t, rp + (size_t)(e / bs) * tr->bytes, row + e, (size_t)n);
      }
      /* each output accumulates the same 256-element chunks in the same order as qvxo_qmatmul */
      for (int v0 = 0; v0 < nvec; v0 += K_VEC_TILE) {
        const int nv = nvec - v0 < K_VEC_TILE ? nvec - v0 : K_VEC_TILE;
        float acc[K_VEC_TILE];
        for (int v = 0; v < nv; ++v) acc[v] = 0.0f;
        for (int e = 0; e < cols; e += per_batch) {
          const int n = cols - e < per_batch ? cols - e : per_batch;
          for (int v = 0; v < nv; ++v) acc[v] += g_dot(row + e, X + (size_t)(v0 + v) * cols + e, n);
        }
        for (int v = 0; v < nv; ++v) out[(size_t)(v0 + v) * rows + r] = acc[v];
      }
    }
    free(row);
  }
  return 1;
}

QVXO_EXPORT int qvxo_dequant_row(const void* weight, uint32_t t, int cols, int row, float* dst) {
  const qvxo_traits* tr = traits_of(t);
  if (!tr || !qvxo_can_dequantize(t)) return 0;
  const int bs = (int)tr->block;
  if (bs <= 0 || cols % bs != 0) return 0;
  const size_t row_bytes = (size_t)(cols / bs) * tr->bytes;
  return qvxo_dequantize(t, (const uint8_t*)weight + (size_t)row * row_bytes, dst, (size_t)cols);
}

/* ---- build-defined oracles ------------------------------------------------------------------ */

/* out[v*rows + r] = sum_k deq(W)[r,k] * X[v,k], dequant values exact in float, summed in double. */
QVXO_EXPORT int qvxo_matmul_f64(double* out, const void* weight, uint32_t t, const float* X, int nvec,
                                int rows, int cols) {
  const qvxo_traits* tr = traits_of(t);
  if (!tr || !qvxo_can_dequantize(t) || nvec <= 0) return 0;
  const int bs = (int)tr->block;
  if (bs <= 0 || cols % bs != 0) return 0;
  const size_t row_bytes = (size_t)(cols / bs) * tr->bytes;
  const uint8_t* base = (const uint8_t*)weight;
#pragma omp parallel
  {
    float* row = (float*)malloc(sizeof(float) * (size_t)(cols > 0 ? cols : 1));
#pragma omp for schedule(static)
    for (int r = 0; r < rows; ++r) {
      qvxo_dequantize(t, base + (size_t)r * row_bytes, row, (size_t)cols);
      for (int v = 0; v < nvec; ++v) {
        const float* x = X + (size_t)v * cols;
        double acc = 0.0;
        for (int k = 0; k < cols; ++k) acc += (double)row[k] * (double)x[k];
        out[(size_t)v * rows + r] = acc;
      }
    }
    free(row);
  }
  return 1;
}

/*
 * Per-32 Q8 activation quantiser (build-defined; the reference has none).  For each row m and
 * block j of 32 values: amax = max|x|, scale = amax / 127 (fp32), q = round-half-away-from-zero
 * (x * (127 / amax)) clamped to [-127, 127]; an all-zero block gets scale 0 and q = 0.
 * Also returns per-block sums of q (int32).  X is fp32 (callers convert fp16 exactly).
 */
QVXO_EXPORT void qvxo_quantize_q8_act(const float* X, int M, int K, int8_t* q, float* scale,
                                      int32_t* qsum) {
  const int nb = K / 32;
  for (int m = 0; m < M; ++m) {
    for (int j = 0; j < nb; ++j) {
      const float* x = X + (size_t)m * K + 32 * j;
      float amax = 0.0f;
      for (int i = 0; i < 32; ++i) amax = fmaxf(amax, fabsf(x[i]));
      const float s = amax / 127.0f;
      const float inv = amax > 0.0f ? 127.0f / amax : 0.0f;
      int32_t sum = 0;
      for (int i = 0; i < 32; ++i) {
        float v = roundf(x[i] * inv);
        if (v > 127.0f) v = 127.0f;
        if (v < -127.0f) v = -127.0f;
        q[(size_t)m * K + 32 * j + i] = (int8_t)v;
        sum += (int32_t)v;
      }
      scale[(size_t)m * nb + j] = s;
      qsum[(size_t)m * nb + j] = sum;
    }
  }
}

/* ---- decoder elementwise ops on the path's inputs and outputs ------------------------------- */

/* The reference's ops::rmsnorm (runtime/src/ops.cpp:8-13): the sum of squares in double, the scale
 * 1 / sqrt(sum / n + eps) in double rounded to float, then x * scale * w in float, left to right. */
QVXO_EXPORT void qvxo_rmsnorm(float* out, const float* x, const float* w, int n, float eps) {
  double ss = 0.0;
  for (int i = 0; i < n; ++i) ss += (double)x[i] * (double)x[i];
  const float scale = (float)(1.0 / sqrt(ss / n + (double)eps));
  for (int i = 0; i < n; ++i) out[i] = x[i] * scale * w[i];
}

/* The reference's ops::swiglu (runtime/src/ops.cpp:96-100): out = silu(g) * u in float, with
 * silu(z) = z / (1 + exp(-z)) (float exp). */
QVXO_EXPORT void qvxo_swiglu(float* out, const float* gate, const float* up, int n) {
  for (int i = 0; i < n; ++i) {
    const float z = gate[i];
    out[i] = z / (1.0f + expf(-z)) * up[i];
  }
}
