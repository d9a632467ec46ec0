// qvx_synth.hip -- seeded synthetic GGUF blocks and activations, generated on the device.
//
// Benchmark and test data only (no reference counterpart).  Every random quantity is a pure
// function of (seed, position) through the SplitMix64 finaliser, so a weight of any size is
// reproducible, generated at HBM speed, and needs no host staging.  Distributions follow the
// benchmark configurations: fp16 scales |N(0,1)| * mul, uniform quant bytes (which makes the
// Q4_K / Q5_K 6-bit scale/min fields and the Q6_K 6-bit quants exactly uniform), Q8_0 quants uniform in
// [-127, 127], Q6_K int8 sub-scales uniform in [-128, 127].
#include "qvx_common.hpp"

namespace qvx {

__device__ inline float u01(uint64_t h) {  // (0, 1], 24 random bits
  return ((float)(uint32_t)(h >> 40) + 1.0f) * (1.0f / 16777216.0f);
}

// Box-Muller: N(0,1) from two uniforms (the cosine branch only).
__device__ inline float normal_at(uint64_t seed, uint64_t i) {
  const uint64_t h1 = splitmix64(seed ^ splitmix64(2 * i));
  const uint64_t h2 = splitmix64(seed ^ splitmix64(2 * i + 1));
  const float r = sqrtf(-2.0f * logf(u01(h1)));
  return r * cospif(2.0f * u01(h2));
}

__device__ inline uint16_t f16_bits(float v) {
  return __builtin_bit_cast(uint16_t, (_Float16)v);
}

// One thread per block.  `blk` counts blocks over the whole tensor (row-major).
template <uint32_t T, int BB>
__global__ __launch_bounds__(256) void k_fill_blocks(uint8_t* __restrict__ w, size_t nblk, uint64_t seed, float mul) {
  const size_t blk = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (blk >= nblk) return;
  uint8_t* p = w + blk * BB;
  const uint64_t s = splitmix64(seed + 0x51ED2701ull * (uint64_t)T);
  auto byte_at = [&](int i) -> uint8_t { return (uint8_t)(splitmix64(s ^ (blk * 256 + (uint64_t)i)) >> 32); };
  auto put16 = [&](int off, uint16_t v) {
    p[off] = (uint8_t)(v & 0xFF);
    p[off + 1] = (uint8_t)(v >> 8);
  };
  if constexpr (T == T_Q8_0) {
    put16(0, f16_bits(fabsf(normal_at(s, 2 * blk)) * mul));
    for (int i = 0; i < 32; ++i) {
      const uint32_t r = (uint32_t)(splitmix64(s ^ (blk * 256 + (uint64_t)i)) >> 32);
      p[2 + i] = (uint8_t)(int8_t)((int)(r % 255u) - 127);
    }
  } else if constexpr (T == T_Q4_0) {
    put16(0, f16_bits(fabsf(normal_at(s, 2 * blk)) * mul));
    for (int i = 0; i < 16; ++i) p[2 + i] = byte_at(i);
  } else if constexpr (T == T_Q4_K || T == T_Q5_K) {
    put16(0, f16_bits(fabsf(normal_at(s, 2 * blk)) * mul));
    put16(2, f16_bits(fabsf(normal_at(s, 2 * blk + 1)) * mul));
    for (int i = 4; i < BB; ++i) p[i] = byte_at(i);
  } else if constexpr (T == T_Q6_K) {
    for (int i = 0; i < 208; ++i) p[i] = byte_at(i);  // ql, qh, and int8 scales uniform
    put16(208, f16_bits(fabsf(normal_at(s, 2 * blk)) * mul));
  }
}

__global__ __launch_bounds__(256) void k_fill_normal_f32(float* __restrict__ x, size_t n, uint64_t seed, float mul) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) x[i] = normal_at(seed, i) * mul;
}

__global__ __launch_bounds__(256) void k_fill_normal_f16(uint16_t* __restrict__ x, size_t n, uint64_t seed, float mul) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) x[i] = f16_bits(normal_at(seed, i) * mul);
}

bool launch_fill_synthetic(void* w, uint32_t t, size_t nblk, uint64_t seed, float mul, hipStream_t s) {
  const unsigned grid = (unsigned)((nblk + 255) / 256);
  auto* p = static_cast<uint8_t*>(w);
  if (nblk == 0) return true;
  switch (t) {
    case T_Q8_0: k_fill_blocks<T_Q8_0, 34><<<grid, 256, 0, s>>>(p, nblk, seed, mul); return true;
    case T_Q4_0: k_fill_blocks<T_Q4_0, 18><<<grid, 256, 0, s>>>(p, nblk, seed, mul); return true;
    case T_Q4_K: k_fill_blocks<T_Q4_K, 144><<<grid, 256, 0, s>>>(p, nblk, seed, mul); return true;
    case T_Q5_K: k_fill_blocks<T_Q5_K, 176><<<grid, 256, 0, s>>>(p, nblk, seed, mul); return true;
    case T_Q6_K: k_fill_blocks<T_Q6_K, 210><<<grid, 256, 0, s>>>(p, nblk, seed, mul); return true;
    default: return false;
  }
}

void launch_fill_normal_f32(float* x, size_t n, uint64_t seed, float mul, hipStream_t s) {
  if (n) k_fill_normal_f32<<<(unsigned)((n + 255) / 256), 256, 0, s>>>(x, n, seed, mul);
}

void launch_fill_normal_f16(uint16_t* x, size_t n, uint64_t seed, float mul, hipStream_t s) {
  if (n) k_fill_normal_f16<<<(unsigned)((n + 255) / 256), 256, 0, s>>>(x, n, seed, mul);
}

// Bare streaming read (benchmark only): one 16-byte load per thread, the fastest pattern measured for
// a single launch on this part.  The loaded words are kept live by a comparison that holds only for
// a fixed pattern (all four words equal to 0x5A17C0DE), in which case the thread stores 1 to *flag;
// any other data writes nothing.
__global__ __launch_bounds__(1024) void k_read16(const uint4* __restrict__ src, size_t n16, uint32_t* __restrict__ flag) {
  const size_t i = (size_t)blockIdx.x * 1024 + threadIdx.x;
  if (i >= n16) return;
  const uint4 v = src[i];
  if ((v.x & v.y & v.z & v.w) == 0x5A17C0DEu && (v.x | v.y | v.z | v.w) == 0x5A17C0DEu) *flag = 1u;
}

void launch_read16(const void* src, size_t n16, uint32_t* flag, hipStream_t s) {
  if (n16) k_read16<<<(unsigned)((n16 + 1023) / 1024), 1024, 0, s>>>(static_cast<const uint4*>(src), n16, flag);
}

}  // namespace qvx
