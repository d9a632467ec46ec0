// qvx_common.hpp -- ggml type table and device helpers shared by the qvx HIP kernels (gfx950).
#pragma once

#include <hip/hip_runtime.h>

#include <atomic>
#include <cstddef>
#include <cstdint>

namespace qvx {

// On-disk ggml type ids (public GGUF format; gguf/include/qorvix/gguf/gguf_types.hpp:17-45).
enum : uint32_t {
  T_F32 = 0,
  T_F16 = 1,
  T_Q4_0 = 2,
  T_Q4_1 = 3,
  T_Q5_0 = 6,
  T_Q5_1 = 7,
  T_Q8_0 = 8,
  T_Q8_1 = 9,
  T_Q4_K = 12,
  T_Q5_K = 13,
  T_Q6_K = 14,
  T_BF16 = 30,
};

struct TypeInfo {
  uint32_t id, block, bytes;
};

// Elements / bytes per block of every id the GGUF format defines (gguf/src/gguf_types.cpp:15-45).
inline constexpr TypeInfo kTypeTable[] = {
    {0, 1, 4},      {1, 1, 2},      {2, 32, 18},    {3, 32, 20},    {6, 32, 22},    {7, 32, 24},
    {8, 32, 34},    {9, 32, 36},    {10, 256, 84},  {11, 256, 110}, {12, 256, 144}, {13, 256, 176},
    {14, 256, 210}, {15, 256, 292}, {16, 256, 66},  {17, 256, 74},  {18, 256, 98},  {19, 256, 50},
    {20, 32, 18},   {21, 256, 110}, {22, 256, 82},  {23, 256, 136}, {24, 1, 1},     {25, 1, 2},
    {26, 1, 4},     {27, 1, 8},     {28, 1, 8},     {29, 256, 56},  {30, 1, 2},
};

inline const TypeInfo* type_info(uint32_t t) {
  for (const auto& e : kTypeTable)
    if (e.id == t) return &e;
  return nullptr;
}

// Types whose dequantisation this engine implements (the reference's canDequantize set).
inline bool can_dequantize(uint32_t t) {
  switch (t) {
    case T_F32: case T_F16: case T_BF16: case T_Q8_0: case T_Q8_1: case T_Q4_0: case T_Q4_1:
    case T_Q5_0: case T_Q5_1: case T_Q4_K: case T_Q5_K: case T_Q6_K:
      return true;
    default:
      return false;
  }
}

// Types the GEMV / GEMM kernels compute.
// Every type the reference's qmatmul accepts (qmatmulSupports = canDequantize && traits,
// runtime/src/qmatmul.cpp:24-26): Q8_0 / Q4_0 / Q4_K / Q6_K on the fast kernels, the others on the
// generic kernel.
inline bool gemv_supports(uint32_t t) { return can_dequantize(t); }

// Block geometry of the four GEMV formats.  A "panel" is PB consecutive blocks of a row: 2048
// elements, PB*BB bytes, always a multiple of 16 so panels of 16-byte-aligned rows stay aligned.
template <uint32_t T> struct Fmt;
template <> struct Fmt<T_Q8_0> { static constexpr int QK = 32, BB = 34, PB = 64; };
template <> struct Fmt<T_Q4_0> { static constexpr int QK = 32, BB = 18, PB = 64; };
template <> struct Fmt<T_Q4_K> { static constexpr int QK = 256, BB = 144, PB = 8; };
template <> struct Fmt<T_Q6_K> { static constexpr int QK = 256, BB = 210, PB = 8; };

// ---- device helpers -------------------------------------------------------------------------

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));

// Exact IEEE half -> single by bit manipulation (subnormals normalised, Inf/NaN payload kept),
// the definition the reference's fp16ToFloat follows (runtime/src/dequant.cpp:222-248).
__host__ __device__ inline float f16_bits_to_f32(uint32_t h) {
  uint32_t sign = (h & 0x8000u) << 16;
  uint32_t e = (h >> 10) & 0x1Fu;
  uint32_t m = h & 0x3FFu;
  uint32_t bits;
  if (e == 0) {
    if (m == 0) {
      bits = sign;
    } else {
      uint32_t fe = 113;
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
  return __builtin_bit_cast(float, bits);
}

// Hardware half -> single for finite values (exact, subnormals included).
__device__ inline float f16lo(uint32_t w) {
  return (float)__builtin_bit_cast(half2_t, w).x;
}
__device__ inline float f16hi(uint32_t w) {
  return (float)__builtin_bit_cast(half2_t, w).y;
}

// ((hi:lo) >> 8*s)[31:0] for s in 0..3: realigns a byte stream read as aligned dwords.
__device__ inline uint32_t align_bytes(uint32_t hi, uint32_t lo, uint32_t s) {
  return __builtin_amdgcn_alignbyte(hi, lo, s);
}

// LDS per compute unit on gfx950: a workgroup's static plus dynamic LDS must fit in it, or the
// dispatch fails at run time (HSA_STATUS_ERROR_INVALID_ALLOCATION) instead of at the launch call.
constexpr int kMaxDevices = 64;
constexpr size_t kLdsPerCU = 160 * 1024;
constexpr size_t kLdsDefaultDyn = 64 * 1024;  // dynamic LDS a kernel may take without raising its limit

// One member of a grouped GEMV launch: out = W . x for the launch's shared vector x.
struct GemvMember {
  const void* w;
  float* y;
  uint32_t type;
  int rows;
  size_t row_bytes;
};

// Per-kernel launch state: the kernel's static LDS (read once from its code object) and the
// dynamic-LDS limit already set on each device (the attribute persists, so hipFuncSetAttribute runs
// only when the limit has to grow: a decode loop does not pay for it on every launch).
struct LdsLimit {
  std::atomic<long> stat{-1};
  std::atomic<int> have[kMaxDevices] = {};
};

// Readies a launch of `kern` with `dyn` bytes of dynamic LDS on the current device.  Returns false,
// and the caller launches nothing, when static + dynamic LDS would exceed the CU's 160 KiB or the
// runtime refuses to report the kernel's attributes or to raise its dynamic limit.
inline bool lds_ready(const void* kern, LdsLimit& lim, size_t dyn) {
  long st = lim.stat.load(std::memory_order_relaxed);
  if (st < 0) {
    hipFuncAttributes a{};
    if (hipFuncGetAttributes(&a, kern) != hipSuccess) return false;
    st = (long)a.sharedSizeBytes;
    lim.stat.store(st, std::memory_order_relaxed);
  }
  if ((size_t)st + dyn > kLdsPerCU) return false;
  if (dyn <= kLdsDefaultDyn) return true;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return false;
  int cur = lim.have[dev].load(std::memory_order_relaxed);
  if (cur >= (int)dyn) return true;
  if (hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)dyn) != hipSuccess) return false;
  while (cur < (int)dyn && !lim.have[dev].compare_exchange_weak(cur, (int)dyn, std::memory_order_relaxed)) {
  }
  return true;
}

// Deterministic K-split epilogue of the GEMM kernels.  The S workgroups of one output tile (grid z =
// split 0..S-1) each store their NA accumulators per thread to part[z][a][thread] (the tile's
// S * NA * nthr floats); the one that arrives last at the tile's counter adds them in split order
// 0, 1, ..., S-1 into acc and returns true: it stores the tile.  The others return false and exit.
// No workgroup waits for another.  Every split must call this (an empty K range stores zeros), and
// the counters start at zero; they end at zero too (the arrival is a wrapping increment whose limit
// is S - 1, so the last split's arrival resets the tile's counter), so a counter block that was
// cleared once serves any number of launches in stream order.  `last` is one int of LDS that no wave still reads (a word of a
// staging buffer once the K loop is over).
// Visibility across the XCDs' separate L2 caches without flushing or invalidating them (a
// device-scope fence writes back and drops the whole L2, which costs the tiles still running their
// K loop far more than this epilogue): the partials are written and read with device-scope relaxed
// atomic accesses, which the compiler issues coherent at device scope (sc1), so each store reaches
// the device-coherent level when it completes and each load reads from it.  Every wave waits for its
// partial stores to complete (s_waitcnt vmcnt(0), an asm statement with a memory clobber, so the
// compiler keeps every store above it) before the barrier after which the counter is incremented (a
// device-scope atomic), and the last split issues its loads only after that atomic has returned.  No
// release / acquire fence is needed on top: completion of a coherent store is the point at which
// other XCDs can see it, and the counter's atomic is ordered after those completions by the wait and
// the barrier; the loads are ordered after the atomic by its returned value (a data dependence
// through the LDS flag and the second barrier).
template <int NA, int NTHR>
__device__ __forceinline__ bool split_k_last(float (&acc)[NA], float* __restrict__ part, uint32_t* cnt, int S,
                                             int z, int tid, int* last) {
  constexpr size_t kSplit = (size_t)NA * NTHR;
  float* mine = part + (size_t)z * kSplit;  // uniform base: lane offsets stay 32-bit
#pragma unroll
  for (int a = 0; a < NA; ++a)
    __hip_atomic_store(mine + (a * NTHR + tid), acc[a], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (tid == 0)
    *last = __builtin_amdgcn_atomic_inc32(cnt, (uint32_t)(S - 1), __ATOMIC_RELAXED, "agent") == (uint32_t)(S - 1);
  __syncthreads();
  if (!*last) return false;
  // Every partial (this split's too) is read back, so acc is free while the sum builds up in it, in
  // split order.  The loads of a split go out CH at a time (CH <= 64 accumulators) and are
  // waited for together: one memory round trip per split and chunk.  (16 at a time, the sums took
  // NA / 16 round trips per split, which slowed a 4-way split at M = 128; all NA at once raised a
  // 128-accumulator kernel past the registers of two waves a SIMD.)
  static_assert(NA % 16 == 0, "accumulators come in 16s");
  constexpr int CH = NA <= 64 ? NA : NA % 64 == 0 ? 64 : NA % 48 == 0 ? 48 : 16;
  static_assert(NA % CH == 0, "whole chunks");
  auto ld = [&](int zz, int a) {
    return __hip_atomic_load(part + (size_t)zz * kSplit + (a * NTHR + tid), __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
  };
#pragma unroll
  for (int a0 = 0; a0 < NA; a0 += CH) {
#pragma unroll
    for (int a = 0; a < CH; ++a) acc[a0 + a] = ld(0, a0 + a);
    for (int zz = 1; zz < S; ++zz) {
      float t[CH];
#pragma unroll
      for (int a = 0; a < CH; ++a) t[a] = ld(zz, a0 + a);
#pragma unroll
      for (int a = 0; a < CH; ++a) acc[a0 + a] += t[a];
    }
  }
  return true;
}

// SplitMix64 finaliser (Steele, Lea, Flood 2014): a counter-based 64-bit hash for seeded data.
__host__ __device__ inline uint64_t splitmix64(uint64_t z) {
  z += 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

}  // namespace qvx
