// qvx_norm.hpp -- RMSNorm and SwiGLU pieces the GEMV kernels fold into their activation prologue and
// their output epilogue (gfx950).
//
// The decoder around the operator normalises the activations before a projection and gates the
// FFN after one (runtime/src/text_model.cpp:146-149,161-165):
//   rmsnorm(x)[i] = x[i] * scale * w[i],  scale = 1 / sqrt(sum x^2 / n + eps)   (ops.cpp:8-13)
//   swiglu(g, u)  = silu(g) * u,           silu(z) = z / (1 + exp(-z))            (ops.cpp:96-100)
// A GEMV workgroup reads every activation of its vectors anyway (each one converts the whole row to
// fixed point), so it can take the sum of squares on the way and normalise before converting.
// Every route -- these kernels and the standalone qvx_rmsnorm -- forms the sum in one canonical
// order, so a vector's scale has the same bits whichever kernel and batch size a call takes:
//  * the row is cut into chunks of 512 elements; lane i of the wave that sums chunk c squares
//    elements 512c + 8i .. +7 in element order (norm_sq8, missing elements past n add nothing);
//  * a chunk's 64 lane sums are combined by the fixed tree of wave_sum64, the chunk sums in chunk
//    order, and the scale is then formed in double as the reference forms it.
// The Q4_K matrix-core kernels' conversion tasks are already 8 consecutive elements dealt in element
// order (with 512 | n each wave of tasks is one chunk); the integer-dot kernel reads the chunks anew.
#pragma once

#include "qvx_common.hpp"

#include <type_traits>

namespace qvx {

// Elements per chunk (one wave of conversion tasks) and the most chunks a vector may have.
constexpr int kNormChunk = 512;
constexpr int kNormMaxChunks = 32;  // n <= 16384

// Sum of the squares of 8 elements, in element order.
__device__ inline float norm_sq8(const float4& a, const float4& b) {
  float s = a.x * a.x;
  s = __builtin_fmaf(a.y, a.y, s);
  s = __builtin_fmaf(a.z, a.z, s);
  s = __builtin_fmaf(a.w, a.w, s);
  s = __builtin_fmaf(b.x, b.x, s);
  s = __builtin_fmaf(b.y, b.y, s);
  s = __builtin_fmaf(b.z, b.z, s);
  s = __builtin_fmaf(b.w, b.w, s);
  return s;
}

// Sum over the 64 lanes of a wave by a fixed balanced tree (pairs, quads, eights, sixteens, rows
// of 32, halves); only commutative adds, so every lane ends with the same bits.
__device__ inline float wave_sum64(float s) {
  auto dpp = [](float v, auto ctrl) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v),
                                                                 decltype(ctrl)::value, 0xF, 0xF, false));
  };
  s += dpp(s, std::integral_constant<int, 0xB1>{});   // quad_perm [1,0,3,2]
  s += dpp(s, std::integral_constant<int, 0x4E>{});   // quad_perm [2,3,0,1]
  s += dpp(s, std::integral_constant<int, 0x141>{});  // row_half_mirror
  s += dpp(s, std::integral_constant<int, 0x140>{});  // row_mirror
  const auto a = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(int, s), __builtin_bit_cast(int, s), false, false);
  s = __builtin_bit_cast(float, (int)a[0]) + __builtin_bit_cast(float, (int)a[1]);
  const auto b = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(int, s), __builtin_bit_cast(int, s), false, false);
  return __builtin_bit_cast(float, (int)b[0]) + __builtin_bit_cast(float, (int)b[1]);
}

// LDS store / load of the chunk sums through inline asm, like the kernels' other LDS traffic in
// their prologue: the compiler cannot tell these addresses from the tile stages that in-flight
// buffer_load ... lds copies write, and would wait for every copy before an access it emits.
__device__ inline void norm_store(uint32_t addr, float v) {
  asm volatile("ds_write_b32 %0, %1" ::"v"(addr), "v"(v) : "memory");
}

// The scale from a vector's chunk sums (LDS at addr, 16-byte aligned, chunk order), as the
// reference forms it: in double, rounded once to float.
__device__ inline float norm_scale(uint32_t addr, int nch, int n, float eps) {
  typedef float f32x4_t __attribute__((ext_vector_type(4)));
  float ss = 0.0f;
  for (int c = 0; c < nch; c += 4) {
    f32x4_t r;
    asm volatile("ds_read_b128 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(r) : "v"(addr + 4u * (uint32_t)c) : "memory");
    ss += r[0];
    if (c + 1 < nch) ss += r[1];
    if (c + 2 < nch) ss += r[2];
    if (c + 3 < nch) ss += r[3];
  }
  return (float)(1.0 / __builtin_sqrt((double)ss / (double)n + (double)eps));
}

// x[i] * scale * w[i], left to right, for a task's 8 elements.
__device__ inline void norm_apply(float4& a, float4& b, float scale, const float4& wa, const float4& wb) {
  a.x = a.x * scale * wa.x;
  a.y = a.y * scale * wa.y;
  a.z = a.z * scale * wa.z;
  a.w = a.w * scale * wa.w;
  b.x = b.x * scale * wb.x;
  b.y = b.y * scale * wb.y;
  b.z = b.z * scale * wb.z;
  b.w = b.w * scale * wb.w;
}

__device__ inline float silu_mul(float g, float u) { return g / (1.0f + expf(-g)) * u; }

// Epilogue/prologue flags of the fused GEMV kernels.
enum : int { EPI_NORM = 1, EPI_SWIGLU = 2 };

// What a fused call adds to the plain product (host side).
struct GemvEpi {
  const float* norm_w = nullptr;  // non-null: the activations are rmsnorm(x, norm_w, eps)
  float eps = 0.0f;
  bool swiglu = false;  // weight rows interleaved in 16-row (gate, up) groups; out = silu(gate) * up
  const float* bias = nullptr;  // non-null (plain calls only): out = W . x + bias, the add last
  bool no_alloc = false;  // the call must not take stream-ordered temporaries (graph-captured plans)
  void* ws = nullptr;     // non-null: workspace the caller owns for the forms that take one
  size_t ws_bytes = 0;
  uint32_t* cnt = nullptr;  // non-null: cnt_n counters, zero on entry, to be left zero (a plan's)
  int cnt_n = 0;
  int flags() const { return (norm_w ? EPI_NORM : 0) | (swiglu ? EPI_SWIGLU : 0); }
};

}  // namespace qvx
