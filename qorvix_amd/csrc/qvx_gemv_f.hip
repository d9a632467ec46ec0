// qvx_gemv_f.hip -- GEMV over unquantised weights (F32, F16, BF16) on gfx950.
//
// out[v, r] = sum_k W[r, k] * X[v, k]: the reference's qmatmul / qmatmulN for the float types it
// accepts (runtime/src/qmatmul.cpp:28-115 over dequant.cpp's F32 copy, fp16ToFloat and bf16ToFloat,
// dequant.cpp:222-255).  Each weight value widens to fp32 exactly; products and sums are fp32 FMAs.
//
// Streaming form: one workgroup of 16 waves per CU, NV vectors of activations staged once into LDS
// as fp32.  A wave takes whole rows; lane l reads 16-byte chunks l, l + 64, ... of the row (8 fp16
// / bf16 or 4 fp32 values), in blocks of U chunks whose loads are all issued before any is used,
// and keeps one fp32 sum per vector: chunks in order, the values of a chunk in order.  The 64 lane
// sums are then combined by a butterfly (xor 32, 16, ..., 1).  A vector's arithmetic does not
// depend on the other vectors of the launch, so qvx_qmatmul_n stays bit-identical to qvx_qmatmul.
#include "qvx_common.hpp"

#include <algorithm>

namespace qvx {

namespace {

constexpr int kU = 8;          // 16-byte chunks per lane per block
constexpr int kCUs = 256;      // MI355X compute units
constexpr size_t kLdsX = 128 * 1024;  // activation staging budget per workgroup

template <uint32_t T>
constexpr int chunk_elems() {
  return T == T_F32 ? 4 : 8;
}

__device__ inline float bf16f(uint32_t h) { return __uint_as_float(h << 16); }

// The chunk's values as fp32, in element order.
template <uint32_t T>
__device__ inline void widen(const uint4 w, float (&f)[chunk_elems<T>()]) {
  if constexpr (T == T_F32) {
    f[0] = __uint_as_float(w.x);
    f[1] = __uint_as_float(w.y);
    f[2] = __uint_as_float(w.z);
    f[3] = __uint_as_float(w.w);
  } else {
    const uint32_t d[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if constexpr (T == T_F16) {
        f[2 * i] = f16lo(d[i]);
        f[2 * i + 1] = f16hi(d[i]);
      } else {
        f[2 * i] = bf16f(d[i] & 0xFFFFu);
        f[2 * i + 1] = bf16f(d[i] >> 16);
      }
    }
  }
}

template <uint32_t T, int NV>
__global__ __launch_bounds__(1024) void k_gemv_float(const uint8_t* __restrict__ W, const float* __restrict__ X,
                                                     float* __restrict__ Y, int rows, int cols, size_t row_bytes) {
  constexpr int E = chunk_elems<T>();
  extern __shared__ float4 xs4[];  // [NV][cols] fp32
  const float* xs = reinterpret_cast<const float*>(xs4);
  const int n4 = NV * cols / 4;
  for (int i = threadIdx.x; i < n4; i += 1024) xs4[i] = reinterpret_cast<const float4*>(X)[i];
  __syncthreads();

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nchunk = cols / E;
  for (int r = blockIdx.x * 16 + wave; r < rows; r += gridDim.x * 16) {
    const uint8_t* rp = W + (size_t)r * row_bytes;
    float acc[NV];
#pragma unroll
    for (int v = 0; v < NV; ++v) acc[v] = 0.0f;
    for (int c0 = 0; c0 < nchunk; c0 += 64 * kU) {
      uint4 w[kU];
#pragma unroll
      for (int u = 0; u < kU; ++u) {
        const int c = c0 + 64 * u + lane;
        w[u] = c < nchunk ? *reinterpret_cast<const uint4*>(rp + (size_t)16 * c) : make_uint4(0, 0, 0, 0);
      }
#pragma unroll
      for (int u = 0; u < kU; ++u) {
        const int c = c0 + 64 * u + lane;
        if (c < nchunk) {
          float f[E];
          widen<T>(w[u], f);
#pragma unroll
          for (int v = 0; v < NV; ++v) {
            const float4* xp = reinterpret_cast<const float4*>(xs + (size_t)v * cols + E * c);
#pragma unroll
            for (int q = 0; q < E / 4; ++q) {
              const float4 x = xp[q];
              acc[v] = __builtin_fmaf(f[4 * q], x.x, acc[v]);
              acc[v] = __builtin_fmaf(f[4 * q + 1], x.y, acc[v]);
              acc[v] = __builtin_fmaf(f[4 * q + 2], x.z, acc[v]);
              acc[v] = __builtin_fmaf(f[4 * q + 3], x.w, acc[v]);
            }
          }
        }
      }
    }
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      float s = acc[v];
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o, 64);
      if (lane == 0) Y[(size_t)v * rows + r] = s;
    }
  }
}

template <uint32_t T, int NV>
bool launch_nv(const uint8_t* w, const float* X, float* Y, int rows, int cols, size_t row_bytes, hipStream_t s) {
  auto kern = &k_gemv_float<T, NV>;
  const size_t lds = (size_t)NV * cols * 4;
  static LdsLimit lim;
  if (!lds_ready(reinterpret_cast<const void*>(kern), lim, lds)) return false;
  const int nwg = (int)std::min<int64_t>(kCUs, ((int64_t)rows + 15) / 16);
  kern<<<(unsigned)nwg, 1024u, lds, s>>>(w, X, Y, rows, cols, row_bytes);
  return true;
}

template <uint32_t T>
bool launch_t(const void* w, const float* X, float* Y, int nvec, int rows, int cols, size_t row_bytes, hipStream_t s) {
  constexpr int E = chunk_elems<T>();
  if (cols % E != 0 || (size_t)cols * 4 > kLdsX) return false;
  const auto* wb = static_cast<const uint8_t*>(w);
  // vectors per launch: as many (1, 2 or 4) as the LDS budget stages
  const int nvmax = (size_t)cols * 16 <= kLdsX ? 4 : (size_t)cols * 8 <= kLdsX ? 2 : 1;
  for (int v0 = 0; v0 < nvec;) {
    const int left = nvec - v0;
    const float* Xv = X + (size_t)v0 * cols;
    float* Yv = Y + (size_t)v0 * rows;
    if (nvmax >= 4 && left >= 4) {
      if (!launch_nv<T, 4>(wb, Xv, Yv, rows, cols, row_bytes, s)) return false;
      v0 += 4;
    } else if (nvmax >= 2 && left >= 2) {
      if (!launch_nv<T, 2>(wb, Xv, Yv, rows, cols, row_bytes, s)) return false;
      v0 += 2;
    } else {
      if (!launch_nv<T, 1>(wb, Xv, Yv, rows, cols, row_bytes, s)) return false;
      v0 += 1;
    }
  }
  return true;
}

}  // namespace

// Float-weight GEMV for 16-byte-aligned weights and activations with 16-byte row pitch.  Returns
// false, having launched nothing, for another type, a row that is not whole 16-byte chunks, or a
// row whose activations do not fit the LDS budget (the generic kernel takes those).
bool launch_gemv_float(uint32_t t, const void* w, const float* X, float* Y, int nvec, int rows, int cols,
                       size_t row_bytes, hipStream_t s) {
  switch (t) {
    case T_F32: return launch_t<T_F32>(w, X, Y, nvec, rows, cols, row_bytes, s);
    case T_F16: return launch_t<T_F16>(w, X, Y, nvec, rows, cols, row_bytes, s);
    case T_BF16: return launch_t<T_BF16>(w, X, Y, nvec, rows, cols, row_bytes, s);
    default: return false;
  }
}

}  // namespace qvx
