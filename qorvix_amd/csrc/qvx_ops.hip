// qvx_ops.hip -- the decoder's elementwise ops on either side of the operator, on gfx950: RMSNorm
// before a projection and SwiGLU after the gate / up projections (runtime/src/text_model.cpp:146-149,
// 161-165).  The fused GEMV kernels fold both into their prologue / epilogue where they can
// (qvx_norm.hpp); these standalone kernels serve every other call and the reference's own entry
// points.
//
//   rmsnorm: out[i] = x[i] * scale * w[i], scale = float(1 / sqrt(sum x^2 / n + eps))
//            (runtime/src/ops.cpp:8-13); the sum in the canonical order of qvx_norm.hpp (the
//            reference sums in double, element by element: the two may differ in the last bit of
//            the scale), the scale in double as the reference forms it
//   swiglu:  out[i] = silu(g[i]) * u[i], silu(z) = z / (1 + exp(-z)) in float (ops.cpp:96-100)
// qvx_common.hpp (hip_runtime.h) must come first: a standard header included before it stops the
// host stubs of template kernels from being emitted.
#include "qvx_common.hpp"
#include "qvx_norm.hpp"

namespace qvx {

namespace {

constexpr int kNormThreads = 1024;

// One workgroup per vector, the canonical order of qvx_norm.hpp: wave w sums chunks w, w + 16, ...
// (lane i: elements 512c + 8i .. +7), the chunk sums go to LDS, then every thread forms the scale
// from them in chunk order and scales its elements.  n up to 16384 (32 chunks).
__global__ __launch_bounds__(kNormThreads) void k_rmsnorm(float* __restrict__ out, const float* __restrict__ x,
                                                          const float* __restrict__ w, int n, float eps) {
  __shared__ __attribute__((aligned(16))) float chunk[kNormMaxChunks];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const float* xv = x + (size_t)blockIdx.x * n;
  float* ov = out + (size_t)blockIdx.x * n;
  const int nch = (n + kNormChunk - 1) / kNormChunk;
  const uint32_t base = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) float*)chunk;
  for (int c = wave; c < nch; c += kNormThreads / 64) {
    float e[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int i = kNormChunk * c + 8 * lane + j;
      e[j] = i < n ? xv[i] : 0.0f;
    }
    const float s = wave_sum64(norm_sq8(make_float4(e[0], e[1], e[2], e[3]), make_float4(e[4], e[5], e[6], e[7])));
    if (lane == 0) norm_store(base + 4u * (uint32_t)c, s);
  }
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
  __builtin_amdgcn_s_barrier();
  const float scale = norm_scale(base, nch, n, eps);
  for (int i = tid; i < n; i += kNormThreads) ov[i] = xv[i] * scale * w[i];
}

__global__ __launch_bounds__(256) void k_swiglu(float* __restrict__ out, const float* __restrict__ g,
                                                const float* __restrict__ u, size_t n) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) out[i] = silu_mul(g[i], u[i]);
}

// SwiGLU of a product over a gate|up weight interleaved in 16-row groups: y holds [nvec][2 ffn]
// (gate rows 32k .. 32k + 15, up rows 32k + 16 .. 32k + 31 for k = 0 ..), out [nvec][ffn].
__global__ __launch_bounds__(256) void k_swiglu_il(float* __restrict__ out, const float* __restrict__ y, int ffn,
                                                   size_t n) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  const size_t v = i / (size_t)ffn, j = i % (size_t)ffn;
  const float* yv = y + v * 2 * (size_t)ffn;
  const size_t g = 32 * (j / 16) + j % 16;
  out[i] = silu_mul(yv[g], yv[g + 16]);
}

// out[v, r] += bias[r]: the reference's bias add after the product (runtime/include/qorvix/runtime/
// weights.hpp:58-80, one fp32 add per output), for the routes whose kernels do not fold it in.
__global__ __launch_bounds__(256) void k_add_bias(float* __restrict__ out, const float* __restrict__ bias, int rows,
                                                  size_t n) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  out[i] += bias[i % (size_t)rows];
}

inline unsigned blocks256(size_t n) { return (unsigned)((n + 255) / 256); }

}  // namespace

void launch_add_bias(float* out, const float* bias, int nvec, int rows, hipStream_t s) {
  const size_t n = (size_t)nvec * (size_t)rows;
  if (n) k_add_bias<<<blocks256(n), 256, 0, s>>>(out, bias, rows, n);
}

void launch_rmsnorm(float* out, const float* x, const float* w, float eps, int nvec, int n, hipStream_t s) {
  k_rmsnorm<<<(unsigned)nvec, kNormThreads, 0, s>>>(out, x, w, n, eps);
}

void launch_swiglu(float* out, const float* g, const float* u, size_t n, hipStream_t s) {
  k_swiglu<<<blocks256(n), 256, 0, s>>>(out, g, u, n);
}

void launch_swiglu_interleaved(float* out, const float* y, int nvec, int ffn, hipStream_t s) {
  const size_t n = (size_t)nvec * (size_t)ffn;
  k_swiglu_il<<<blocks256(n), 256, 0, s>>>(out, y, ffn, n);
}

}  // namespace qvx
