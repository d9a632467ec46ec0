// qvx_dequant.hip -- GGUF block dequantisation to fp32 on gfx950, bit-exact with the reference.
//
// Whole blocks from a 4-byte-aligned source into a 16-byte-aligned output: each workgroup copies its
// 2048 elements' blocks into LDS with coalesced dword loads, then each thread decodes eight
// consecutive elements from LDS and stores them as 16-byte vectors.  Otherwise one thread per output
// element decodes its element from its block's bytes in global memory (block headers re-read by
// neighbouring threads and served from L1).  Every formula is the public ggml block definition as the
// reference states it in runtime/src/dequant.cpp:38-210; the products are exact in fp32, so the
// single rounding (Q4_K / Q5_K subtract, Q4_1 / Q5_1 add) gives the same value in any order.
#include "qvx_deq.hpp"

namespace qvx {

// dst[i] = dequant(src)[i] for i < n; QK / BB are the type's block geometry.
template <uint32_t T, int QK, int BB>
__global__ __launch_bounds__(256) void k_dequant(const uint8_t* __restrict__ src, float* __restrict__ dst,
                                                 size_t n) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  const size_t blk = i / QK;
  const int e = (int)(i - blk * QK);
  dst[i] = deq_elem<T>(src + blk * BB, e);
}

__global__ __launch_bounds__(256) void k_copy_f32(const uint32_t* __restrict__ src, uint32_t* __restrict__ dst,
                                                  size_t n) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) dst[i] = src[i];
}

// Eight consecutive elements e0 .. e0 + 7 (e0 % 8 == 0) of one block in LDS, decoded with the block's
// header read once: they always share one scale (Q8_0 / Q4_0: the block's, Q4_K: one 32-element
// sub-block's, Q6_K: one 16-element scale group's).  Same formulas and operand order as deq_elem; the
// fp16 scales are converted by the hardware (exact for every finite value, subnormals included).
__device__ inline uint32_t lds_u32_at(const uint8_t* p) {  // 4 bytes at any address, from aligned dwords
  const uintptr_t a = reinterpret_cast<uintptr_t>(p);
  const uint32_t* w = reinterpret_cast<const uint32_t*>(a & ~(uintptr_t)3);
  return align_bytes(w[1], w[0], (uint32_t)(a & 3));
}
__device__ inline float f16at(const uint8_t* p) {
  const uintptr_t a = reinterpret_cast<uintptr_t>(p);  // 2-byte aligned
  const uint32_t w = *reinterpret_cast<const uint32_t*>(a & ~(uintptr_t)3);
  return (a & 2) ? f16hi(w) : f16lo(w);
}

template <uint32_t T>
__device__ inline void deq8(const uint8_t* b, int e0, float (&v)[8]) {
#pragma unroll
  for (int k = 0; k < 8; ++k) v[k] = deq_elem<T>(b, e0 + k);
}
template <>
__device__ inline void deq8<T_Q8_0>(const uint8_t* b, int e0, float (&v)[8]) {
  const float d = f16at(b);
  const uint32_t w0 = lds_u32_at(b + 2 + e0), w1 = lds_u32_at(b + 6 + e0);
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    v[k] = d * (float)(int8_t)(w0 >> (8 * k));
    v[4 + k] = d * (float)(int8_t)(w1 >> (8 * k));
  }
}
template <>
__device__ inline void deq8<T_Q4_0>(const uint8_t* b, int e0, float (&v)[8]) {
  const float d = f16at(b);
  const int o = e0 & 15, sh = e0 < 16 ? 0 : 4;
  const uint32_t w0 = lds_u32_at(b + 2 + o) >> sh, w1 = lds_u32_at(b + 6 + o) >> sh;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    v[k] = (float)((int)((w0 >> (8 * k)) & 15u) - 8) * d;
    v[4 + k] = (float)((int)((w1 >> (8 * k)) & 15u) - 8) * d;
  }
}
template <>
__device__ inline void deq8<T_Q4_K>(const uint8_t* b, int e0, float (&v)[8]) {
  const int c = e0 >> 6, l = e0 & 63, hi = l >> 5;
  uint32_t sc, m;
  k4_scale_min(2 * c + hi, b + 4, sc, m);
  const float ds = f16at(b) * (float)sc;
  const float dm = f16at(b + 2) * (float)m;
  const int sh = hi ? 4 : 0;
  const uint32_t* q = reinterpret_cast<const uint32_t*>(b + 16 + 32 * c + (l & 31));  // 4-byte aligned
  const uint32_t w0 = q[0] >> sh, w1 = q[1] >> sh;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    v[k] = ds * (float)((w0 >> (8 * k)) & 15u) - dm;
    v[4 + k] = ds * (float)((w1 >> (8 * k)) & 15u) - dm;
  }
}
template <>
__device__ inline void deq8<T_Q6_K>(const uint8_t* b, int e0, float (&v)[8]) {
  const int h = e0 >> 7, p = e0 & 127, quarter = p >> 5, l = p & 31;
  const uint32_t a0 = lds_u32_at(b + 64 * h + l + 32 * (quarter & 1));
  const uint32_t a1 = lds_u32_at(b + 64 * h + l + 32 * (quarter & 1) + 4);
  const uint32_t h0 = lds_u32_at(b + 128 + 32 * h + l), h1 = lds_u32_at(b + 128 + 32 * h + l + 4);
  const int nsh = (quarter & 2) ? 4 : 0, hsh = 2 * quarter;
  const float d = f16at(b + 208);
  const float ds = d * (float)(int8_t)b[192 + 8 * h + (l >> 4) + 2 * quarter];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int q0 = (int)(((a0 >> (8 * k + nsh)) & 15u) | (((h0 >> (8 * k + hsh)) & 3u) << 4));
    const int q1 = (int)(((a1 >> (8 * k + nsh)) & 15u) | (((h1 >> (8 * k + hsh)) & 3u) << 4));
    v[k] = ds * (float)(q0 - 32);
    v[4 + k] = ds * (float)(q1 - 32);
  }
}

constexpr int kStageElems = 2048;  // elements per workgroup of the LDS-staged kernels

// Copies workgroup blockIdx.x's blocks (elements [2048 x, 2048 x + 2048) of n, whole blocks) into sm
// with dword loads, the tensor's last partial dword byte by byte; ends with a barrier.
template <int QK, int BB>
__device__ inline void stage_blocks(const uint8_t* __restrict__ src, size_t n, uint32_t* sm) {
  constexpr int kBytes = kStageElems / QK * BB;
  static_assert(kStageElems % QK == 0 && kBytes % 4 == 0, "workgroup span must be whole blocks and dwords");
  const int tid = threadIdx.x;
  const size_t b0 = (size_t)blockIdx.x * kStageElems / QK * BB;
  const size_t avail = min((size_t)kBytes, n / QK * BB - b0);
  const uint32_t* g4 = reinterpret_cast<const uint32_t*>(src + b0);
  for (int k = tid; k < (int)(avail / 4); k += 256) sm[k] = g4[k];
  const int full = (int)(avail & ~(size_t)3);
  if (tid < (int)(avail & 3)) reinterpret_cast<uint8_t*>(sm)[full + tid] = src[b0 + full + tid];
  __syncthreads();
}

// fp32 output: dst[i] = dequant(src)[i] from the staged blocks (dst 16-byte aligned), stored so that
// a wave's store covers 1 KiB contiguous.  Q4_0 / Q4_K / Q5_K: eight consecutive elements a thread
// (one 32-element group: the block header, or the 6-bit scale and min, decoded once for the eight)
// into LDS, then stored from there.  The other formats: four consecutive elements a thread per round
// (4t .. 4t + 3, then 1024 + 4t ..), one 16-byte store each.  Measured on MI355X against two 16-byte
// stores of eight elements a thread (graph-timed, weights cycled): Q4_K 14336 x 4096 73 -> 55.5 us,
// Q4_0 11008 x 4096 51 -> 47, Q8_0 4096 x 4096 19.9 -> 16.4, Q6_K 4096 x 14336 73 -> 64; Q8_0 and
// Q6_K on the eight-element form with LDS took 18.7 and 72.
template <uint32_t T, int QK, int BB>
__global__ __launch_bounds__(256) void k_dequant_lds(const uint8_t* __restrict__ src, float4* __restrict__ dst,
                                                     size_t n) {
  __shared__ uint32_t sm[kStageElems / QK * BB / 4];
  stage_blocks<QK, BB>(src, n, sm);
  const int tid = threadIdx.x;
  if constexpr (T == T_Q4_0 || T == T_Q4_K || T == T_Q5_K) {
    // eight elements a thread into LDS, then the span stored as 1 KiB a wave
    __shared__ float4 ob[kStageElems / 4];
    const uint8_t* b = reinterpret_cast<const uint8_t*>(sm) + (8 * tid) / QK * BB;
    const int e = (8 * tid) % QK;
    float v[8];
    if constexpr (T != T_Q5_K) {
      deq8<T>(b, e, v);  // deq_elem's formulas and operand order, the block header decoded once
    } else {
#pragma unroll
      for (int k = 0; k < 8; ++k) v[k] = deq_elem<T>(b, e + k);
    }
    ob[2 * tid] = make_float4(v[0], v[1], v[2], v[3]);
    ob[2 * tid + 1] = make_float4(v[4], v[5], v[6], v[7]);
    __syncthreads();
#pragma unroll
    for (int r = 0; r < kStageElems / 1024; ++r) {
      const size_t i = (size_t)blockIdx.x * kStageElems + 1024 * r + 4 * tid;
      if (i < n) dst[i / 4] = ob[256 * r + tid];
    }
  } else {
#pragma unroll
    for (int r = 0; r < kStageElems / 1024; ++r) {
      const int e0 = 1024 * r + 4 * tid;  // four elements of one block (every block size is a multiple of 4)
      const size_t i = (size_t)blockIdx.x * kStageElems + e0;
      if (i >= n) break;
      const uint8_t* b = reinterpret_cast<const uint8_t*>(sm) + e0 / QK * BB;
      const int e = e0 % QK;
      dst[i / 4] = make_float4(deq_elem<T>(b, e), deq_elem<T>(b, e + 1), deq_elem<T>(b, e + 2), deq_elem<T>(b, e + 3));
    }
  }
}

// Host launcher: returns false for a type outside the dequantisable set.
bool launch_dequant(uint32_t t, const void* src, float* dst, size_t n, hipStream_t s) {
  const size_t grid = (n + 255) / 256;
  if (n == 0) return true;
  const auto* b = static_cast<const uint8_t*>(src);
  // block types over whole blocks, source 4-byte and destination 16-byte aligned: staged through LDS
  const size_t qk = (t == T_Q4_K || t == T_Q5_K || t == T_Q6_K) ? 256 : 32;
  if (t != T_F32 && t != T_F16 && t != T_BF16 && n % qk == 0 && (reinterpret_cast<uintptr_t>(src) & 3u) == 0 &&
      (reinterpret_cast<uintptr_t>(dst) & 15u) == 0) {
    const unsigned g = (unsigned)((n + kStageElems - 1) / kStageElems);
    auto* d4 = reinterpret_cast<float4*>(dst);
    switch (t) {
      case T_Q8_0: k_dequant_lds<T_Q8_0, 32, 34><<<g, 256, 0, s>>>(b, d4, n); return true;
      case T_Q8_1: k_dequant_lds<T_Q8_1, 32, 36><<<g, 256, 0, s>>>(b, d4, n); return true;
      case T_Q4_0: k_dequant_lds<T_Q4_0, 32, 18><<<g, 256, 0, s>>>(b, d4, n); return true;
      case T_Q4_1: k_dequant_lds<T_Q4_1, 32, 20><<<g, 256, 0, s>>>(b, d4, n); return true;
      case T_Q5_0: k_dequant_lds<T_Q5_0, 32, 22><<<g, 256, 0, s>>>(b, d4, n); return true;
      case T_Q5_1: k_dequant_lds<T_Q5_1, 32, 24><<<g, 256, 0, s>>>(b, d4, n); return true;
      case T_Q4_K: k_dequant_lds<T_Q4_K, 256, 144><<<g, 256, 0, s>>>(b, d4, n); return true;
      case T_Q5_K: k_dequant_lds<T_Q5_K, 256, 176><<<g, 256, 0, s>>>(b, d4, n); return true;
      case T_Q6_K: k_dequant_lds<T_Q6_K, 256, 210><<<g, 256, 0, s>>>(b, d4, n); return true;
      default: return false;
    }
  }
  switch (t) {
    case T_F32: k_copy_f32<<<grid, 256, 0, s>>>((const uint32_t*)src, (uint32_t*)dst, n); return true;
    case T_F16: k_dequant<T_F16, 1, 2><<<grid, 256, 0, s>>>(b, dst, n); return true;
    case T_BF16: k_dequant<T_BF16, 1, 2><<<grid, 256, 0, s>>>(b, dst, n); return true;
    case T_Q8_0: k_dequant<T_Q8_0, 32, 34><<<grid, 256, 0, s>>>(b, dst, n); return true;
    case T_Q8_1: k_dequant<T_Q8_1, 32, 36><<<grid, 256, 0, s>>>(b, dst, n); return true;
    case T_Q4_0: k_dequant<T_Q4_0, 32, 18><<<grid, 256, 0, s>>>(b, dst, n); return true;
    case T_Q4_1: k_dequant<T_Q4_1, 32, 20><<<grid, 256, 0, s>>>(b, dst, n); return true;
    case T_Q5_0: k_dequant<T_Q5_0, 32, 22><<<grid, 256, 0, s>>>(b, dst, n); return true;
    case T_Q5_1: k_dequant<T_Q5_1, 32, 24><<<grid, 256, 0, s>>>(b, dst, n); return true;
    case T_Q4_K: k_dequant<T_Q4_K, 256, 144><<<grid, 256, 0, s>>>(b, dst, n); return true;
    case T_Q5_K: k_dequant<T_Q5_K, 256, 176><<<grid, 256, 0, s>>>(b, dst, n); return true;
    case T_Q6_K: k_dequant<T_Q6_K, 256, 210><<<grid, 256, 0, s>>>(b, dst, n); return true;
    default: return false;
  }
}

// ---- dequantisation to 16-bit (prefill GEMM operands) ----------------------------------------------
// The fp32 value above, rounded once to nearest-even fp16 or bf16 (NaN stays NaN, quiet).
__device__ inline uint16_t to_bf16(float f) {
  const uint32_t u = __builtin_bit_cast(uint32_t, f);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 0x0040u);
  return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

// fp32 -> fp16 bits, round to nearest even.  The value is pinned first: otherwise the compiler folds
// the product that produced it and the conversion into one mixed-precision multiply-add with a +0
// addend, which turns a -0 product (a zero code times a negative scale) into +0.
__device__ inline uint16_t to_f16(float f) {
  asm volatile("" : "+v"(f));
  return __builtin_bit_cast(uint16_t, (_Float16)f);
}

template <uint32_t T, int QK, int BB, bool BF>
__global__ __launch_bounds__(256) void k_dequant16(const uint8_t* __restrict__ src, uint16_t* __restrict__ dst,
                                                   size_t n) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  float v;
  if constexpr (T == T_F32) {
    v = reinterpret_cast<const float*>(src)[i];
  } else {
    const size_t blk = i / QK;
    v = deq_elem<T>(src + blk * BB, (int)(i - blk * QK));
  }
  dst[i] = BF ? to_bf16(v) : to_f16(v);
}

// Eight consecutive elements per thread (always inside one block: every block size is a multiple
// of 8), so the block header is read once for the eight and the result leaves as one 16-byte store.
template <uint32_t T, int QK, int BB, bool BF>
__global__ __launch_bounds__(256) void k_dequant16x8(const uint8_t* __restrict__ src, uint4* __restrict__ dst,
                                                     size_t n8) {
  const size_t g = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (g >= n8) return;
  const size_t i = 8 * g;
  float v[8];
  if constexpr (T == T_F32) {
    const float4* p = reinterpret_cast<const float4*>(src) + 2 * g;
    const float4 a = p[0], c = p[1];
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = c.x; v[5] = c.y; v[6] = c.z; v[7] = c.w;
  } else {
    const size_t blk = i / QK;
    const int e = (int)(i - blk * QK);
    const uint8_t* b = src + blk * BB;
#pragma unroll
    for (int k = 0; k < 8; ++k) v[k] = deq_elem<T>(b, e + k);
  }
  uint32_t w[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t lo = BF ? to_bf16(v[2 * j]) : to_f16(v[2 * j]);
    const uint32_t hi = BF ? to_bf16(v[2 * j + 1]) : to_f16(v[2 * j + 1]);
    w[j] = lo | (hi << 16);
  }
  dst[g] = make_uint4(w[0], w[1], w[2], w[3]);
}

// Block types, staged: a workgroup's 2048 elements are whole blocks (2048 / QK of them, a multiple
// of 4 bytes in every format), copied from a 4-byte-aligned source into LDS with coalesced dword
// loads (the last partial dword of the tensor byte by byte), then each thread dequantises eight
// consecutive elements from LDS as above.  n is a whole number of blocks.
template <uint32_t T, int QK, int BB, bool BF>
__global__ __launch_bounds__(256) void k_dequant16_lds(const uint8_t* __restrict__ src, uint4* __restrict__ dst,
                                                       size_t n) {
  __shared__ uint32_t sm[kStageElems / QK * BB / 4];
  stage_blocks<QK, BB>(src, n, sm);
  const int tid = threadIdx.x;
  const size_t i = (size_t)blockIdx.x * kStageElems + 8 * (size_t)tid;
  if (i >= n) return;
  const uint8_t* b = reinterpret_cast<const uint8_t*>(sm) + (8 * tid) / QK * BB;
  const int e = (8 * tid) % QK;
  float v[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) v[k] = deq_elem<T>(b, e + k);
  uint32_t w[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t lo = BF ? to_bf16(v[2 * j]) : to_f16(v[2 * j]);
    const uint32_t hi = BF ? to_bf16(v[2 * j + 1]) : to_f16(v[2 * j + 1]);
    w[j] = lo | (hi << 16);
  }
  dst[i / 8] = make_uint4(w[0], w[1], w[2], w[3]);
}

// ---- 16-bit dequantisation, wide workgroups -------------------------------------------------------
constexpr int kWideElems = 8192;  // elements per workgroup of the wide 16-bit dequantiser

// A workgroup's 8192 elements are whole blocks; their bytes (a multiple of 16 in every block format at
// this size) are copied from a 16-byte-aligned source into LDS with 16-byte loads (the tensor's last
// bytes one at a time), then each thread decodes eight consecutive elements per round, four rounds,
// and stores them as one 16-byte vector (a wave stores 1 KiB contiguous).  n: whole blocks.
// The body for workgroup wg (the standalone kernel passes blockIdx.x).
template <uint32_t T, int QK, int BB, bool BF>
__device__ __forceinline__ void dequant16_wide_body(const uint8_t* __restrict__ src, uint4* __restrict__ dst, size_t n,
                                                    unsigned wg) {
  constexpr int kBytes = kWideElems / QK * BB;
  static_assert(kWideElems % QK == 0 && kBytes % 16 == 0, "workgroup span must be whole blocks and 16-byte units");
  __shared__ __attribute__((aligned(16))) uint32_t sm[kBytes / 4 + 4];
  const int tid = threadIdx.x;
  const size_t b0 = (size_t)wg * kBytes;
  const size_t avail = min((size_t)kBytes, n / QK * BB - b0);
  const uint4* g16 = reinterpret_cast<const uint4*>(src + b0);
  for (int k = tid; k < (int)(avail / 16); k += 256) reinterpret_cast<uint4*>(sm)[k] = g16[k];
  const int full = (int)(avail & ~(size_t)15);
  if (tid < (int)(avail & 15)) reinterpret_cast<uint8_t*>(sm)[full + tid] = src[b0 + full + tid];
  __syncthreads();
  const uint8_t* sb = reinterpret_cast<const uint8_t*>(sm);
#pragma unroll
  for (int r = 0; r < kWideElems / 2048; ++r) {
    const int e0 = r * 2048 + 8 * tid;
    const size_t i = (size_t)wg * kWideElems + e0;
    if (i >= n) break;
    float v[8];
    deq8<T>(sb + (e0 / QK) * BB, e0 % QK, v);
    uint32_t w[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t lo = BF ? to_bf16(v[2 * j]) : to_f16(v[2 * j]);
      const uint32_t hi = BF ? to_bf16(v[2 * j + 1]) : to_f16(v[2 * j + 1]);
      w[j] = lo | (hi << 16);
    }
    dst[i / 8] = make_uint4(w[0], w[1], w[2], w[3]);
  }
}

template <uint32_t T, int QK, int BB, bool BF>
__global__ __launch_bounds__(256) void k_dequant16_wide(const uint8_t* __restrict__ src, uint4* __restrict__ dst,
                                                        size_t n) {
  dequant16_wide_body<T, QK, BB, BF>(src, dst, n, blockIdx.x);
}

// The wide dequantiser (bf16) and the bf16 rounding of the GEMM's fp16 activations in one launch:
// workgroups [0, nwg) take the weight as k_dequant16_wide does, the rest convert x (n8 groups of
// 8 values, four groups a thread in a grid-stride loop) as the 16-bit GEMM's own prepass does
// (round to nearest even, NaN kept quiet), so the two memory-bound passes share one launch.
template <uint32_t T, int QK, int BB>
__global__ __launch_bounds__(256) void k_dequant16_wide_x(const uint8_t* __restrict__ src, uint4* __restrict__ dst,
                                                          size_t n, unsigned nwg, const uint4* __restrict__ x,
                                                          uint4* __restrict__ xo, size_t n8) {
  if (blockIdx.x < nwg) {
    dequant16_wide_body<T, QK, BB, true>(src, dst, n, blockIdx.x);
    return;
  }
  auto cv = [](uint32_t w) {
    const uint32_t lo = to_bf16((float)__builtin_bit_cast(_Float16, (uint16_t)(w & 0xFFFFu)));
    const uint32_t hi = to_bf16((float)__builtin_bit_cast(_Float16, (uint16_t)(w >> 16)));
    return lo | (hi << 16);
  };
  const size_t stride = (size_t)(gridDim.x - nwg) * 256;
  for (size_t i = (size_t)(blockIdx.x - nwg) * 256 + threadIdx.x; i < n8; i += stride) {
    const uint4 v = x[i];
    xo[i] = make_uint4(cv(v.x), cv(v.y), cv(v.z), cv(v.w));
  }
}

template <bool BF>
bool launch_dequant16_wide(uint32_t t, const uint8_t* b, uint4* d8, size_t n, hipStream_t s) {
  const unsigned grid = (unsigned)((n + kWideElems - 1) / kWideElems);
  switch (t) {
    case T_Q8_0: k_dequant16_wide<T_Q8_0, 32, 34, BF><<<grid, 256, 0, s>>>(b, d8, n); return true;
    case T_Q4_0: k_dequant16_wide<T_Q4_0, 32, 18, BF><<<grid, 256, 0, s>>>(b, d8, n); return true;
    case T_Q5_0: k_dequant16_wide<T_Q5_0, 32, 22, BF><<<grid, 256, 0, s>>>(b, d8, n); return true;
    case T_Q4_K: k_dequant16_wide<T_Q4_K, 256, 144, BF><<<grid, 256, 0, s>>>(b, d8, n); return true;
    case T_Q5_K: k_dequant16_wide<T_Q5_K, 256, 176, BF><<<grid, 256, 0, s>>>(b, d8, n); return true;
    case T_Q6_K: k_dequant16_wide<T_Q6_K, 256, 210, BF><<<grid, 256, 0, s>>>(b, d8, n); return true;
    default: return false;
  }
}

// The weight of n elements to bf16 and x (n8 groups of 8 fp16 values, 16-byte aligned) to bf16 in
// one launch; false, having launched nothing, where the wide kernel does not take the weight.
bool launch_dequant16_bf16_x(uint32_t t, const void* src, uint16_t* dst, size_t n, const uint16_t* x, uint16_t* xo,
                             size_t n8, hipStream_t s) {
  const size_t qk = (t == T_Q4_K || t == T_Q5_K || t == T_Q6_K) ? 256 : 32;
  if (n == 0 || n % qk != 0 || (reinterpret_cast<uintptr_t>(src) & 15u) || (reinterpret_cast<uintptr_t>(dst) & 15u) ||
      (reinterpret_cast<uintptr_t>(x) & 15u) || (reinterpret_cast<uintptr_t>(xo) & 15u))
    return false;
  const unsigned nwg = (unsigned)((n + kWideElems - 1) / kWideElems);
  const unsigned nx = (unsigned)std::min<size_t>((n8 + 1023) / 1024, 4096);
  const dim3 grid(nwg + nx);
  const auto* b = static_cast<const uint8_t*>(src);
  auto* d8 = reinterpret_cast<uint4*>(dst);
  const auto* x8 = reinterpret_cast<const uint4*>(x);
  auto* o8 = reinterpret_cast<uint4*>(xo);
  switch (t) {
    case T_Q8_0: k_dequant16_wide_x<T_Q8_0, 32, 34><<<grid, 256, 0, s>>>(b, d8, n, nwg, x8, o8, n8); return true;
    case T_Q4_0: k_dequant16_wide_x<T_Q4_0, 32, 18><<<grid, 256, 0, s>>>(b, d8, n, nwg, x8, o8, n8); return true;
    case T_Q5_0: k_dequant16_wide_x<T_Q5_0, 32, 22><<<grid, 256, 0, s>>>(b, d8, n, nwg, x8, o8, n8); return true;
    case T_Q4_K: k_dequant16_wide_x<T_Q4_K, 256, 144><<<grid, 256, 0, s>>>(b, d8, n, nwg, x8, o8, n8); return true;
    case T_Q5_K: k_dequant16_wide_x<T_Q5_K, 256, 176><<<grid, 256, 0, s>>>(b, d8, n, nwg, x8, o8, n8); return true;
    case T_Q6_K: k_dequant16_wide_x<T_Q6_K, 256, 210><<<grid, 256, 0, s>>>(b, d8, n, nwg, x8, o8, n8); return true;
    default: return false;
  }
}

template <bool BF>
bool launch_dequant16_lds(uint32_t t, const uint8_t* b, uint4* d8, size_t n, hipStream_t s) {
  const unsigned grid = (unsigned)((n + kStageElems - 1) / kStageElems);
  switch (t) {
    case T_Q8_0: k_dequant16_lds<T_Q8_0, 32, 34, BF><<<grid, 256, 0, s>>>(b, d8, n); return true;
    case T_Q8_1: k_dequant16_lds<T_Q8_1, 32, 36, BF><<<grid, 256, 0, s>>>(b, d8, n); return true;
    case T_Q4_0: k_dequant16_lds<T_Q4_0, 32, 18, BF><<<grid, 256, 0, s>>>(b, d8, n); return true;
    case T_Q4_1: k_dequant16_lds<T_Q4_1, 32, 20, BF><<<grid, 256, 0, s>>>(b, d8, n); return true;
    case T_Q5_0: k_dequant16_lds<T_Q5_0, 32, 22, BF><<<grid, 256, 0, s>>>(b, d8, n); return true;
    case T_Q5_1: k_dequant16_lds<T_Q5_1, 32, 24, BF><<<grid, 256, 0, s>>>(b, d8, n); return true;
    case T_Q4_K: k_dequant16_lds<T_Q4_K, 256, 144, BF><<<grid, 256, 0, s>>>(b, d8, n); return true;
    case T_Q5_K: k_dequant16_lds<T_Q5_K, 256, 176, BF><<<grid, 256, 0, s>>>(b, d8, n); return true;
    case T_Q6_K: k_dequant16_lds<T_Q6_K, 256, 210, BF><<<grid, 256, 0, s>>>(b, d8, n); return true;
    default: return false;
  }
}

template <bool BF>
bool launch_dequant16_t(uint32_t t, const void* src, uint16_t* dst, size_t n, hipStream_t s) {
  if (n == 0) return true;
  const auto* b = static_cast<const uint8_t*>(src);
  // block types over whole blocks: the LDS-staged kernel (source 4-byte, destination 16-byte aligned)
  const size_t qk = (t == T_Q4_K || t == T_Q5_K || t == T_Q6_K) ? 256 : 32;
  // the wide kernel: 16-byte-aligned source and destination
  if (t != T_F32 && t != T_F16 && t != T_BF16 && n % qk == 0 && (reinterpret_cast<uintptr_t>(src) & 15u) == 0 &&
      (reinterpret_cast<uintptr_t>(dst) & 15u) == 0 &&
      launch_dequant16_wide<BF>(t, b, reinterpret_cast<uint4*>(dst), n, s))
    return true;
  if (t != T_F32 && t != T_F16 && t != T_BF16 && n % qk == 0 && (reinterpret_cast<uintptr_t>(src) & 3u) == 0 &&
      (reinterpret_cast<uintptr_t>(dst) & 15u) == 0 &&
      launch_dequant16_lds<BF>(t, b, reinterpret_cast<uint4*>(dst), n, s))
    return true;
  // whole groups of 8 on the vector kernel (dst 16-byte aligned; F32 sources too), the rest scalar
  const bool vec = (reinterpret_cast<uintptr_t>(dst) & 15u) == 0 &&
                   (t != T_F32 || (reinterpret_cast<uintptr_t>(src) & 15u) == 0);
  const size_t n8 = vec ? n / 8 : 0;
  if (n8) {
    const size_t grid8 = (n8 + 255) / 256;
    auto* d8 = reinterpret_cast<uint4*>(dst);
    switch (t) {
      case T_F32: k_dequant16x8<T_F32, 1, 4, BF><<<grid8, 256, 0, s>>>(b, d8, n8); break;
      case T_F16: k_dequant16x8<T_F16, 1, 2, BF><<<grid8, 256, 0, s>>>(b, d8, n8); break;
      case T_BF16: k_dequant16x8<T_BF16, 1, 2, BF><<<grid8, 256, 0, s>>>(b, d8, n8); break;
      case T_Q8_0: k_dequant16x8<T_Q8_0, 32, 34, BF><<<grid8, 256, 0, s>>>(b, d8, n8); break;
      case T_Q8_1: k_dequant16x8<T_Q8_1, 32, 36, BF><<<grid8, 256, 0, s>>>(b, d8, n8); break;
      case T_Q4_0: k_dequant16x8<T_Q4_0, 32, 18, BF><<<grid8, 256, 0, s>>>(b, d8, n8); break;
      case T_Q4_1: k_dequant16x8<T_Q4_1, 32, 20, BF><<<grid8, 256, 0, s>>>(b, d8, n8); break;
      case T_Q5_0: k_dequant16x8<T_Q5_0, 32, 22, BF><<<grid8, 256, 0, s>>>(b, d8, n8); break;
      case T_Q5_1: k_dequant16x8<T_Q5_1, 32, 24, BF><<<grid8, 256, 0, s>>>(b, d8, n8); break;
      case T_Q4_K: k_dequant16x8<T_Q4_K, 256, 144, BF><<<grid8, 256, 0, s>>>(b, d8, n8); break;
      case T_Q5_K: k_dequant16x8<T_Q5_K, 256, 176, BF><<<grid8, 256, 0, s>>>(b, d8, n8); break;
      case T_Q6_K: k_dequant16x8<T_Q6_K, 256, 210, BF><<<grid8, 256, 0, s>>>(b, d8, n8); break;
      default: return false;
    }
  }
  const size_t done = 8 * n8;
  if (done == n) return true;
  // the tail: whole blocks for the quantised types (n is a whole number of blocks), so the scalar
  // kernel indexes from a block boundary; F32 / F16 / BF16 have one-element blocks
  const TypeInfo* ti = type_info(t);
  if (!ti) return false;
  b += done / ti->block * ti->bytes;
  dst += done;
  n -= done;
  const size_t grid = (n + 255) / 256;
  switch (t) {
    case T_F32: k_dequant16<T_F32, 1, 4, BF><<<grid, 256, 0, s>>>(b, dst, n); return true;
    case T_F16: k_dequant16<T_F16, 1, 2, BF><<<grid, 256, 0, s>>>(b, dst, n); return true;
    case T_BF16: k_dequant16<T_BF16, 1, 2, BF><<<grid, 256, 0, s>>>(b, dst, n); return true;
    case T_Q8_0: k_dequant16<T_Q8_0, 32, 34, BF><<<grid, 256, 0, s>>>(b, dst, n); return true;
    case T_Q8_1: k_dequant16<T_Q8_1, 32, 36, BF><<<grid, 256, 0, s>>>(b, dst, n); return true;
    case T_Q4_0: k_dequant16<T_Q4_0, 32, 18, BF><<<grid, 256, 0, s>>>(b, dst, n); return true;
    case T_Q4_1: k_dequant16<T_Q4_1, 32, 20, BF><<<grid, 256, 0, s>>>(b, dst, n); return true;
    case T_Q5_0: k_dequant16<T_Q5_0, 32, 22, BF><<<grid, 256, 0, s>>>(b, dst, n); return true;
    case T_Q5_1: k_dequant16<T_Q5_1, 32, 24, BF><<<grid, 256, 0, s>>>(b, dst, n); return true;
    case T_Q4_K: k_dequant16<T_Q4_K, 256, 144, BF><<<grid, 256, 0, s>>>(b, dst, n); return true;
    case T_Q5_K: k_dequant16<T_Q5_K, 256, 176, BF><<<grid, 256, 0, s>>>(b, dst, n); return true;
    case T_Q6_K: k_dequant16<T_Q6_K, 256, 210, BF><<<grid, 256, 0, s>>>(b, dst, n); return true;
    default: return false;
  }
}

// dst[i] = 16-bit rounding of dequant(src)[i] (bf16 when `bf16`, else fp16), i < n.
bool launch_dequant16(uint32_t t, const void* src, uint16_t* dst, size_t n, bool bf16, hipStream_t s) {
  return bf16 ? launch_dequant16_t<true>(t, src, dst, n, s) : launch_dequant16_t<false>(t, src, dst, n, s);
}

// ---- generic GEMV: any alignment, any supported type ---------------------------------------------
// One wave per (row, vector); lane-strided elements dequantised with deq_elem; used only when a
// weight's base or row pitch is not 16-byte aligned (the fast kernels in qvx_gemv.hip need both).
// Bit-identity across n_vec holds here too: each output is the same lane sums and the same tree.
template <uint32_t T, int QK, int BB>
__global__ __launch_bounds__(256) void k_gemv_generic(const uint8_t* __restrict__ W, const float* __restrict__ X,
                                                      float* __restrict__ Y, int rows, int cols, int nvec,
                                                      size_t row_bytes) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const long task = (long)blockIdx.x * 4 + wave;
  if (task >= (long)rows * nvec) return;
  const int v = (int)(task / rows), r = (int)(task - (long)v * rows);
  const uint8_t* rp = W + (size_t)r * row_bytes;
  const float* x = X + (size_t)v * cols;
  float acc = 0.0f;
  for (int k = lane; k < cols; k += 64) {
    const int blk = k / QK;
    float w;
    if constexpr (T == T_F32)
      w = ((const float*)rp)[k];
    else
      w = deq_elem<T>(rp + (size_t)blk * BB, k - blk * QK);
    acc = __builtin_fmaf(w, x[k], acc);
  }
  for (int off = 32; off > 0; off >>= 1) acc += __shfl_xor(acc, off, 64);
  if (lane == 0) Y[(size_t)v * rows + r] = acc;
}

// Runs of eight: one wave per row, up to NV vectors a pass; lane l takes the runs of eight
// consecutive elements l, l + 64, ... (a run never crosses a block: every block size is 1 or a
// multiple of 8), decodes each weight element once for all NV vectors, and keeps one fp32 sum per
// vector, runs in order and elements in order within a run, then the same xor tree.  A vector's
// arithmetic does not depend on NV or on the other vectors, so batched calls stay bit-identical to
// single ones.  Needs cols % 8 == 0 and 16-byte-aligned activations.
template <uint32_t T, int QK, int BB, int NV>
__global__ __launch_bounds__(256) void k_gemv_generic8(const uint8_t* __restrict__ W, const float* __restrict__ X,
                                                       float* __restrict__ Y, int rows, int cols, int nvec,
                                                       size_t row_bytes) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int r = blockIdx.x * 4 + wave;
  if (r >= rows) return;
  const uint8_t* rp = W + (size_t)r * row_bytes;
  const int nrun = cols / 8;
  for (int v0 = 0; v0 < nvec; v0 += NV) {
    const int nv = min(NV, nvec - v0);
    float acc[NV];
#pragma unroll
    for (int v = 0; v < NV; ++v) acc[v] = 0.0f;
    for (int g = lane; g < nrun; g += 64) {
      const int k = 8 * g;
      float w[8];
      if constexpr (T == T_F32) {
#pragma unroll
        for (int e = 0; e < 8; ++e) w[e] = reinterpret_cast<const float*>(rp)[k + e];
      } else {
        const int blk = k / QK;
        const uint8_t* bp = rp + (size_t)blk * BB;
#pragma unroll
        for (int e = 0; e < 8; ++e) w[e] = deq_elem<T>(bp + (QK == 1 ? 2 * e : 0), QK == 1 ? 0 : k - blk * QK + e);
      }
#pragma unroll
      for (int v = 0; v < NV; ++v) {
        if (v < nv) {
          const float4* xp = reinterpret_cast<const float4*>(X + (size_t)(v0 + v) * cols + k);
          const float4 x0 = xp[0], x1 = xp[1];
          const float xs[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
          for (int e = 0; e < 8; ++e) acc[v] = __builtin_fmaf(w[e], xs[e], acc[v]);
        }
      }
    }
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      float a = acc[v];
      for (int off = 32; off > 0; off >>= 1) a += __shfl_xor(a, off, 64);
      if (v < nv && lane == 0) Y[(size_t)(v0 + v) * rows + r] = a;
    }
  }
}

template <uint32_t T, int QK, int BB>
void launch_generic8(const uint8_t* b, const float* X, float* Y, int rows, int cols, int nvec, size_t row_bytes,
                     hipStream_t s) {
  k_gemv_generic8<T, QK, BB, 4><<<(unsigned)((rows + 3) / 4), 256, 0, s>>>(b, X, Y, rows, cols, nvec, row_bytes);
}

bool launch_gemv_generic(uint32_t t, const void* w, const float* X, float* Y, int rows, int cols, int nvec,
                         size_t row_bytes, hipStream_t s) {
  const auto* b8 = static_cast<const uint8_t*>(w);
  if (cols % 8 == 0 && (reinterpret_cast<uintptr_t>(X) & 15u) == 0 &&
      (t != T_F32 || (reinterpret_cast<uintptr_t>(w) & 3u) == 0)) {
    switch (t) {
      case T_F32: launch_generic8<T_F32, 1, 4>(b8, X, Y, rows, cols, nvec, row_bytes, s); return true;
      case T_F16: launch_generic8<T_F16, 1, 2>(b8, X, Y, rows, cols, nvec, row_bytes, s); return true;
      case T_BF16: launch_generic8<T_BF16, 1, 2>(b8, X, Y, rows, cols, nvec, row_bytes, s); return true;
      case T_Q8_0: launch_generic8<T_Q8_0, 32, 34>(b8, X, Y, rows, cols, nvec, row_bytes, s); return true;
      case T_Q8_1: launch_generic8<T_Q8_1, 32, 36>(b8, X, Y, rows, cols, nvec, row_bytes, s); return true;
      case T_Q4_0: launch_generic8<T_Q4_0, 32, 18>(b8, X, Y, rows, cols, nvec, row_bytes, s); return true;
      case T_Q4_1: launch_generic8<T_Q4_1, 32, 20>(b8, X, Y, rows, cols, nvec, row_bytes, s); return true;
      case T_Q5_0: launch_generic8<T_Q5_0, 32, 22>(b8, X, Y, rows, cols, nvec, row_bytes, s); return true;
      case T_Q5_1: launch_generic8<T_Q5_1, 32, 24>(b8, X, Y, rows, cols, nvec, row_bytes, s); return true;
      case T_Q4_K: launch_generic8<T_Q4_K, 256, 144>(b8, X, Y, rows, cols, nvec, row_bytes, s); return true;
      case T_Q5_K: launch_generic8<T_Q5_K, 256, 176>(b8, X, Y, rows, cols, nvec, row_bytes, s); return true;
      case T_Q6_K: launch_generic8<T_Q6_K, 256, 210>(b8, X, Y, rows, cols, nvec, row_bytes, s); return true;
      default: return false;
    }
  }
  const long tasks = (long)rows * nvec;
  const unsigned grid = (unsigned)((tasks + 3) / 4);
  const auto* b = static_cast<const uint8_t*>(w);
  switch (t) {
    case T_F32: k_gemv_generic<T_F32, 1, 4><<<grid, 256, 0, s>>>(b, X, Y, rows, cols, nvec, row_bytes); return true;
    case T_Q8_0: k_gemv_generic<T_Q8_0, 32, 34><<<grid, 256, 0, s>>>(b, X, Y, rows, cols, nvec, row_bytes); return true;
    case T_Q4_0: k_gemv_generic<T_Q4_0, 32, 18><<<grid, 256, 0, s>>>(b, X, Y, rows, cols, nvec, row_bytes); return true;
    case T_Q4_K: k_gemv_generic<T_Q4_K, 256, 144><<<grid, 256, 0, s>>>(b, X, Y, rows, cols, nvec, row_bytes); return true;
    case T_Q6_K: k_gemv_generic<T_Q6_K, 256, 210><<<grid, 256, 0, s>>>(b, X, Y, rows, cols, nvec, row_bytes); return true;
    case T_F16: k_gemv_generic<T_F16, 1, 2><<<grid, 256, 0, s>>>(b, X, Y, rows, cols, nvec, row_bytes); return true;
    case T_BF16: k_gemv_generic<T_BF16, 1, 2><<<grid, 256, 0, s>>>(b, X, Y, rows, cols, nvec, row_bytes); return true;
    case T_Q8_1: k_gemv_generic<T_Q8_1, 32, 36><<<grid, 256, 0, s>>>(b, X, Y, rows, cols, nvec, row_bytes); return true;
    case T_Q4_1: k_gemv_generic<T_Q4_1, 32, 20><<<grid, 256, 0, s>>>(b, X, Y, rows, cols, nvec, row_bytes); return true;
    case T_Q5_0: k_gemv_generic<T_Q5_0, 32, 22><<<grid, 256, 0, s>>>(b, X, Y, rows, cols, nvec, row_bytes); return true;
    case T_Q5_1: k_gemv_generic<T_Q5_1, 32, 24><<<grid, 256, 0, s>>>(b, X, Y, rows, cols, nvec, row_bytes); return true;
    case T_Q5_K: k_gemv_generic<T_Q5_K, 256, 176><<<grid, 256, 0, s>>>(b, X, Y, rows, cols, nvec, row_bytes); return true;
    default: return false;
  }
}

}  // namespace qvx
