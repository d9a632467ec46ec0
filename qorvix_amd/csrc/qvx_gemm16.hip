// qvx_gemm16.hip -- plain 16-bit matrix-core GEMM on gfx950, and the prefill GEMM of every weight
// type that has no raw-block kernel of its own: the weight dequantised once into 16 bits, then this
// GEMM.
//
// out[m, n] = sum_k X[m, k] * B[n, k],  X [M, K] and B [N, K] bf16 or fp16 row-major, out fp32 with
// row stride ldy.  As the prefill GEMM: B = the reference's exact dequantised weight value
// (runtime/src/dequant.cpp:38-210) rounded once to bf16 / fp16, X the fp16 activations (bf16: rounded
// once); the semantics are qmatmulN's (runtime/src/qmatmul.cpp:64-115) with X converted fp16 -> fp32
// exactly.  The reference has no GEMM (it prefills token by token).
//
// Two kernels: k_gemm16q (below), 256 threads on 256-token x 256-row tiles, for grids that fill the
// chip; and k_gemm16, 8 waves on 128-token tiles with a K split, for the smaller grids.
//
// k_gemm16: workgroup = 512 threads, 8 waves, a BM x 256 output tile (BM = 256 or 128 tokens x 256 weight rows).
// Wave w owns weight rows 64 (w % 4) .. +63 and tokens (BM / 2) (w / 4) .. + BM/2 - 1:
// 2 x BM/64 tiles of v_mfma_f32_32x32x16_{bf16,f16}, accumulators in registers.
// K advances in slices of KS elements (32 at BM = 256, 64 at BM = 128); both operands of a slice are
// copied global -> LDS by buffer_load ... lds (16 bytes a lane, no registers) into a ring of NST
// stages (4 x 32 KiB, or 3 x 48 KiB), NST - 1 slices ahead.  In LDS a row of a slice is KS * 2 bytes
// with its 16-byte chunk c at slot c ^ swz(row), so the fragment reads of 16 consecutive rows (one
// chunk each) hit distinct banks.
//
// Schedule ("ping-pong"): the two waves of a SIMD (w and w + 4) take turns.  The workgroup runs in
// phases separated by barriers; in each phase one group of four waves (one per SIMD) issues the 16
// MFMAs of a slice from fragments already in its registers while the other group issues its copies
// of a later slice, reads its fragments of the next slice from LDS and waits for them.  So each SIMD's
// matrix pipe is fed by one wave while its partner's LDS traffic and copy issue run beside it, and no
// MFMA waits for LDS.  Group 0 reads slice j in phase 2j and multiplies it in phase 2j + 1; group 1
// reads it in phase 2j + 1 and multiplies it in phase 2j + 2.  A slice's stage is overwritten only by
// the copies of slice j + NST, issued once both groups have read slice j (phase >= 2j + 2), and every
// wave waits for its copies of slice j + 1 before the barrier that ends phase 2j + 1.
// Tiles are numbered in a 1-D grid, M-tile fastest within a column of 256 weight rows, consecutive
// numbers on one XCD (the dispatcher deals workgroups round-robin over the 8 XCDs), so the tiles an
// XCD runs at once share their weight rows and X rows in its L2.  Grids smaller than the chip split K
// across workgroups; the split that finishes a tile last adds the partial tiles in split order
// (split_k_last), so results do not vary between runs.
// qvx_common.hpp (hip_runtime.h) must come first: a standard header included before it stops the
// host stubs of template kernels from being emitted.
#include "qvx_common.hpp"

#include <algorithm>

namespace qvx {

namespace g16 {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
#define QVX_LDS __attribute__((address_space(3)))

enum { VAR_BF16 = 0, VAR_F16 = 2 };
constexpr uint32_t kRsrcWord3 = 0x00020000u;  // raw buffer, 32-bit data (gfx9)
constexpr int kBN = 256;                      // weight rows per tile

struct Geo {
  int M, N, K;       // N: the rows of B this launch covers
  int ldy;           // row stride of out (elements)
  int mt;            // M tiles per column of 256 weight rows
  int per_split;     // K slices per workgroup along grid z
  float* part;       // K-split launches: partial tiles [tile][split][BM * 256]
  uint32_t* cnt;     // ... and one arrival counter per tile, zero before the launch
};

// s_waitcnt vmcnt(N), other counters untouched (gfx9 encoding).
template <int N>
__device__ inline void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// LDS reads through inline asm: the compiler cannot tell them from the stages the in-flight
// buffer_load ... lds copies write and would otherwise wait for every copy before each read.  The
// copies are ordered explicitly (wait_vm before a barrier).
template <int OFF>
__device__ inline u32x4 lds_read16(uint32_t addr) {
  u32x4 r;
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "i"(OFF) : "memory");
  return r;
}

// Copy global -> LDS, 16 bytes a lane (a device function of its own: called from a lambda, the target
// builtin makes the host pass drop the kernel's launch stub).
__device__ inline void copy_lds16(__amdgpu_buffer_rsrc_t r, QVX_LDS uint8_t* dst, uint32_t voff, uint32_t soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, dst, 16, voff, soff, 0, 0);
}

// Slot of chunk 0 of row r: rows of 4 chunks (64 bytes) or 8 chunks (128 bytes).
template <int CPR>
__device__ inline uint32_t swz(uint32_t r) {
  if constexpr (CPR == 4)
    return (r >> 2) & 3u;
  else
    return (r ^ ((r >> 3) & 3u)) & 7u;
}

template <int VAR>
__device__ inline f32x16_t mfma32(const u32x4& a, const u32x4& b, f32x16_t c) {
  if constexpr (VAR == VAR_BF16)
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b), c,
                                                   0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a), __builtin_bit_cast(f16x8_t, b), c, 0,
                                                  0, 0);
}

// Waits for every LDS read in flight; the fragments are operands, so no MFMA moves above the wait.
template <int NF>
__device__ inline void lds_wait_all(u32x4 (&f)[NF]);
template <>
__device__ inline void lds_wait_all<6>(u32x4 (&f)[6]) {
  asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(f[0]), "+v"(f[1]), "+v"(f[2]), "+v"(f[3]), "+v"(f[4]), "+v"(f[5])::"memory");
}
template <>
__device__ inline void lds_wait_all<8>(u32x4 (&f)[8]) {
  asm volatile("s_waitcnt lgkmcnt(0)"
               : "+v"(f[0]), "+v"(f[1]), "+v"(f[2]), "+v"(f[3]), "+v"(f[4]), "+v"(f[5]), "+v"(f[6]), "+v"(f[7])::"memory");
}
template <>
__device__ inline void lds_wait_all<12>(u32x4 (&f)[12]) {
  asm volatile("s_waitcnt lgkmcnt(0)"
               : "+v"(f[0]), "+v"(f[1]), "+v"(f[2]), "+v"(f[3]), "+v"(f[4]), "+v"(f[5]), "+v"(f[6]), "+v"(f[7]),
                 "+v"(f[8]), "+v"(f[9]), "+v"(f[10]), "+v"(f[11])::"memory");
}
template <>
__device__ inline void lds_wait_all<16>(u32x4 (&f)[16]) {
  asm volatile("s_waitcnt lgkmcnt(0)"
               : "+v"(f[0]), "+v"(f[1]), "+v"(f[2]), "+v"(f[3]), "+v"(f[4]), "+v"(f[5]), "+v"(f[6]), "+v"(f[7]),
                 "+v"(f[8]), "+v"(f[9]), "+v"(f[10]), "+v"(f[11]), "+v"(f[12]), "+v"(f[13]), "+v"(f[14]),
                 "+v"(f[15])::"memory");
}

}  // namespace g16

using namespace g16;

template <int VAR, int BM, int KS>
__global__ __launch_bounds__(512) void k_gemm16(const uint16_t* __restrict__ X, const uint16_t* __restrict__ B,
                                                float* __restrict__ Y, Geo geo) {
  constexpr int RB = KS * 2;               // LDS bytes of one row of a slice
  constexpr int CPR = KS / 8;              // 16-byte chunks a row
  constexpr int XST = BM * RB;             // X part of a stage
  constexpr int STB = (BM + kBN) * RB;     // one stage: X rows, then B rows
  constexpr int NST = (150 * 1024) / STB;  // stages: 4 (BM 256, KS 32) or 3 (BM 128, KS 64)
  constexpr int CPS = STB / 1024 / 8;      // 1 KiB copies per wave per slice: 4 or 6
  constexpr int XC = XST / 1024;           // copies of a slice that move X
  constexpr int TM = BM / 64;              // 32-token tiles of a wave
  constexpr int TN = 2;                    // 32-row tiles of a wave
  constexpr int ST = KS / 16;              // K16 steps a slice
  constexpr int NF = ST * (TM + TN);       // fragments a wave reads per slice: 12 or 16
  constexpr int YOUNG = (NST - 2) * CPS;   // copies a wave issues after those of the slice it waits for
  static_assert(NST >= 3 && NST * STB <= 160 * 1024, "LDS budget");
  static_assert(NF == 12 || NF == 16, "fragment count");
  __shared__ __attribute__((aligned(1024))) uint8_t lds[NST * STB];

  const int M = geo.M, N = geo.N, K = geo.K;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int grp = wave >> 2, wr = wave & 3;
  const int ln = lane & 31, g = lane >> 5;
  int tile;
  {
    const int nb = (int)gridDim.x;
    int b = (int)blockIdx.x;
    if ((nb & 7) == 0) b = (b & 7) * (nb >> 3) + (b >> 3);  // XCD b % 8 takes a contiguous range
    tile = b;
  }
  const int n0 = (tile / geo.mt) * kBN, m0 = (tile % geo.mt) * BM;
  const int nsl = K / KS;
  const int kb0 = (int)blockIdx.z * geo.per_split;
  const int L = min(nsl, kb0 + geo.per_split) - kb0;  // slices of this split (an empty split stores zeros)
  if (m0 >= M || n0 >= N) return;

  // Copy descriptors: rows past M or N read as zeros (buffer range check).
  const uint32_t row_bytes = (uint32_t)K * 2u;
  const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(X + (size_t)m0 * K), (short)0, (int)((uint32_t)min(BM, M - m0) * row_bytes), (int)kRsrcWord3);
  const __amdgpu_buffer_rsrc_t br = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(B + (size_t)n0 * K), (short)0, (int)((uint32_t)min(kBN, N - n0) * row_bytes), (int)kRsrcWord3);
  // Copy i of this wave moves 1 KiB of a stage: c = wave * CPS + i, chunk q = 64 (c mod X/B) + lane
  // -> row q / CPR, LDS slot q % CPR holds global chunk slot ^ swz(row).  c < XC: X rows, else B rows.
  uint32_t voff[CPS];
  bool isx[CPS];
#pragma unroll
  for (int i = 0; i < CPS; ++i) {
    const int c = wave * CPS + i;
    isx[i] = c < XC;
    const uint32_t q = (uint32_t)((isx[i] ? c : c - XC) * 64 + lane), r = q / CPR, p = q % CPR;
    voff[i] = r * row_bytes + 16u * (p ^ swz<CPR>(r));
  }
  QVX_LDS uint8_t* lds_l = (QVX_LDS uint8_t*)lds;
  auto issue = [&](int j) {  // this wave's copies of slice j (relative to kb0)
    QVX_LDS uint8_t* st = lds_l + (j % NST) * STB + wave * CPS * 1024;
    const uint32_t so = (uint32_t)(kb0 + j) * (uint32_t)RB;
#pragma unroll
    for (int i = 0; i < CPS; ++i) copy_lds16(isx[i] ? xr : br, st + i * 1024, voff[i], so);
  };

  // Fragment addresses: lane (ln, g) reads row ln of a 32-row tile, chunk 2s + g of K16 step s.
  const uint32_t lds_base = (uint32_t)(uintptr_t)lds_l;
  uint32_t frel[ST];
#pragma unroll
  for (int s = 0; s < ST; ++s) frel[s] = (uint32_t)ln * RB + 16u * ((2u * s + (uint32_t)g) ^ swz<CPR>((uint32_t)ln));
  const uint32_t xw = (uint32_t)(grp * (BM / 2)) * RB;  // this wave's token rows in the X part
  const uint32_t bw = (uint32_t)XST + (uint32_t)(wr * 64) * RB;  // its weight rows in the B part

  u32x4 fr[NF];  // [s][TM A tiles, TN B tiles]
  auto read_slice = [&](int j) {
    const uint32_t st = lds_base + (uint32_t)(j % NST) * STB;
#pragma unroll
    for (int s = 0; s < ST; ++s) {
      const uint32_t a = st + xw + frel[s], b = st + bw + frel[s];
      fr[s * (TM + TN) + 0] = lds_read16<0>(a);
      fr[s * (TM + TN) + 1] = lds_read16<32 * RB>(a);
      if constexpr (TM == 4) {
        fr[s * (TM + TN) + 2] = lds_read16<64 * RB>(a);
        fr[s * (TM + TN) + 3] = lds_read16<96 * RB>(a);
      }
      fr[s * (TM + TN) + TM] = lds_read16<0>(b);
      fr[s * (TM + TN) + TM + 1] = lds_read16<32 * RB>(b);
    }
    lds_wait_all<NF>(fr);
  };

  f32x16_t acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int n = 0; n < TN; ++n)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][n][e] = 0.0f;

  auto mfmas = [&]() {
#pragma unroll
    for (int s = 0; s < ST; ++s)
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int n = 0; n < TN; ++n)
          acc[i][n] = mfma32<VAR>(fr[s * (TM + TN) + i], fr[s * (TM + TN) + TM + n], acc[i][n]);
  };
  // Before a barrier: this wave's copies of slice j + 1 complete (steady state: the copies of NST - 2
  // later slices may still fly; near the end fewer were issued, so wait for all).
  auto sync = [&](int j) {
    if (j + NST - 1 < L)
      wait_vm<YOUNG>();
    else
      wait_vm<0>();
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
  };

  // Prologue: slices 0 .. NST - 2 in flight, slice 0 complete.
#pragma unroll
  for (int j = 0; j < NST - 1; ++j)
    if (j < L) issue(j);
  if (NST - 1 <= L)
    wait_vm<YOUNG>();
  else
    wait_vm<0>();
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_sched_barrier(0);
  if (grp == 1) {  // phase 0: group 0 reads slice 0, group 1 has nothing to multiply yet
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
  }
  for (int j = 0; j < L; ++j) {
    // read phase of slice j: copies of slice j + NST - 1 into the stage slice j - 1 held
    if (j + NST - 1 < L) issue(j + NST - 1);
    read_slice(j);
    sync(j);
    // MFMA phase of slice j
    mfmas();
    __builtin_amdgcn_sched_barrier(0);
    if (grp == 0 || j + 1 < L) sync(j);
  }

  // K split: the split that finishes a tile last sums the partials in split order and stores it.
  if (gridDim.z > 1) {
    constexpr int NA = TM * TN * 16;
    float v[NA];
#pragma unroll
    for (int a = 0; a < NA; ++a) v[a] = acc[a / (TN * 16)][(a / 16) % TN][a % 16];
    if (!split_k_last<NA, 512>(v, geo.part + (size_t)tile * gridDim.z * (NA * 512), geo.cnt + tile, (int)gridDim.z,
                               (int)blockIdx.z, tid, reinterpret_cast<int*>(lds)))
      return;
#pragma unroll
    for (int a = 0; a < NA; ++a) acc[a / (TN * 16)][(a / 16) % TN][a % 16] = v[a];
  }

  // C layout of v_mfma_f32_32x32x*: element e of lane l is row 8 (e / 4) + 4 (l / 32) + e % 4 (token),
  // column l % 32 (weight row).
#pragma unroll
  for (int n = 0; n < TN; ++n) {
    const int col = n0 + 64 * wr + 32 * n + ln;
    if (col >= N) continue;
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int m = m0 + grp * (BM / 2) + 32 * i + 8 * (e >> 2) + 4 * g + (e & 3);
        if (m < M) Y[(size_t)m * geo.ldy + col] = acc[i][n][e];
      }
  }
}

// ---- 4-wave form: one wave per SIMD, 128 x 128 wave tiles ------------------------------------------
// k_gemm16q<VAR, BM, KS, NST>: a BM-token x 256-row tile per 256-thread workgroup; wave w owns tokens
// (BM / 2) (w / 2) .. + BM/2 - 1 and weight rows 128 (w % 2) .. +127 (BM / 64 x 4 tiles of
// v_mfma_f32_32x32x16_*; at BM = 256, 256 accumulators held in the accumulation registers).  The
// product runs BM = 256; at BM = 128 this form measured 3-8 % slower than the 8-wave kernel on the
// same tiles, which therefore keeps the 128-token tiles.  Per K16 step a wave reads 8 fragments (8 KiB) for
// 16 MFMAs, two thirds of the LDS traffic per MFMA of the 8-wave form's 64 x 128 wave tiles.  K
// advances in KS-element slices through NST stages (X rows, then B rows, KS * 2 bytes a row, the
// 8-wave form's layout and swizzles), each filled by buffer_load ... lds NST - 1 slices ahead.  The
// product path runs KS = 64 with two 64 KiB stages: a copy then moves whole 128-byte lines of a row
// (32-element slices read each line twice, in two slices, and measured 10 % slower on MI355X at
// 2048 x 14336 x 4096 even with four or five stages).  The wave software-pipelines itself: while the
// 16 MFMAs of one step issue, the fragment reads of the next step issue between them (and, in a
// slice's last step, the copies of slice j + NST and the first reads of slice j + 1), so the matrix
// pipe waits on LDS only when a read is late.  One barrier per slice, before its last step: every
// wave has then read the whole slice (the last step's fragments are in registers), so the slice's
// stage is refilled during that step, and each wave has waited for its copies of slice j + 1 before
// it.  The K order of the products is the 8-wave form's (K16 steps in order into each accumulator),
// so both forms give the same bits.
template <int VAR, int BM, int KS, int NST>
__global__ __launch_bounds__(256) void k_gemm16q(const uint16_t* __restrict__ X, const uint16_t* __restrict__ B,
                                                 float* __restrict__ Y, Geo geo) {
  constexpr int RB = KS * 2, CPR = KS / 8;
  constexpr int XST = BM * RB;           // X part of a stage
  constexpr int STB = XST + kBN * RB;    // one stage: X rows, then B rows
  constexpr int CPS = STB / 1024 / 4;    // 1 KiB copies per wave per slice
  constexpr int XC = XST / 1024;         // copies of a slice that move X
  constexpr int ST = KS / 16;            // K16 steps a slice
  constexpr int TM = BM / 64;            // 32-token tiles of a wave (it covers BM / 2 tokens)
  constexpr int NF = TM + 4;             // fragments a step: TM of X, 4 of B
  constexpr int NS = 4 * TM;             // MFMAs a step
  constexpr int YOUNG = (NST - 2) * CPS;
  static_assert(NST >= 2 && NST * STB <= 160 * 1024, "LDS budget");
  static_assert(ST % 2 == 0 && (BM == 128 || BM == 256), "tile shape");
  __shared__ __attribute__((aligned(1024))) uint8_t lds[NST * STB];
  const int M = geo.M, N = geo.N, K = geo.K;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  const int ln = lane & 31, g = lane >> 5;
  int tile;
  {
    const int nb = (int)gridDim.x;
    int b = (int)blockIdx.x;
    if ((nb & 7) == 0) b = (b & 7) * (nb >> 3) + (b >> 3);  // XCD b % 8 takes a contiguous range
    tile = b;
  }
  const int n0 = (tile / geo.mt) * kBN, m0 = (tile % geo.mt) * BM;
  const int kb0 = 0, L = K / KS;  // no K split: the plan runs this kernel on grids that fill the chip
  if (m0 >= M || n0 >= N) return;
  const uint32_t row_bytes = (uint32_t)K * 2u;
  const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(X + (size_t)m0 * K), (short)0, (int)((uint32_t)min(BM, M - m0) * row_bytes), (int)kRsrcWord3);
  const __amdgpu_buffer_rsrc_t br = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(B + (size_t)n0 * K), (short)0, (int)((uint32_t)min(kBN, N - n0) * row_bytes), (int)kRsrcWord3);
  // Copy i of this wave moves 1 KiB of a stage: c = wave * CPS + i, chunk q = 64 (c mod X / B) + lane
  // -> row q / CPR, LDS slot q % CPR holds global chunk slot ^ swz(row).  c < XC: X rows, else B rows.
  uint32_t voff[CPS];
  bool isx[CPS];
#pragma unroll
  for (int i = 0; i < CPS; ++i) {
    const int c = wave * CPS + i;
    isx[i] = c < XC;
    const uint32_t q = (uint32_t)((isx[i] ? c : c - XC) * 64 + lane), r = q / CPR, p = q % CPR;
    voff[i] = r * row_bytes + 16u * (p ^ swz<CPR>(r));
  }
  QVX_LDS uint8_t* lds_l = (QVX_LDS uint8_t*)lds;
  const uint32_t lds_base = (uint32_t)(uintptr_t)lds_l;
  auto copy1 = [&](int j, int i) {  // copy i of slice j (relative to kb0)
    QVX_LDS uint8_t* st = lds_l + (j % NST) * STB + (wave * CPS + i) * 1024;
    copy_lds16(isx[i] ? xr : br, st, voff[i], (uint32_t)(kb0 + j) * (uint32_t)RB);
  };
  uint32_t frel[ST];
#pragma unroll
  for (int s = 0; s < ST; ++s) frel[s] = (uint32_t)ln * RB + 16u * ((2u * s + (uint32_t)g) ^ swz<CPR>((uint32_t)ln));
  const uint32_t xw = (uint32_t)(wm * (BM / 2)) * RB;
  const uint32_t bw = (uint32_t)XST + (uint32_t)(wn * 128) * RB;
  // Fragment k of step s of slice j: X tiles 0 .. TM - 1, then B tiles 0 .. 3.
  auto read1 = [&](int j, int s, int k) -> u32x4 {
    const bool isa = k < TM;
    const int t = isa ? k : k - TM;
    const uint32_t st = lds_base + (uint32_t)(j % NST) * STB + frel[s] + (isa ? xw : bw);
    switch (t) {
      case 0: return lds_read16<0>(st);
      case 1: return lds_read16<32 * RB>(st);
      case 2: return lds_read16<64 * RB>(st);
      default: return lds_read16<96 * RB>(st);
    }
  };
  f32x16_t acc[TM][4];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int n = 0; n < 4; ++n)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][n][e] = 0.0f;
  u32x4 f[2][NF];
#pragma unroll
  for (int j = 0; j < NST; ++j)
    if (j < L)
#pragma unroll
      for (int i = 0; i < CPS; ++i) copy1(j, i);
  if (L >= NST)
    wait_vm<(NST - 1) * CPS>();
  else
    wait_vm<0>();
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int k = 0; k < NF; ++k) f[0][k] = read1(0, 0, k);
  lds_wait_all<NF>(f[0]);
  // One slice; REFILL: the copies of slice j + NST are issued, MORE: slice j + 1 follows.  In every
  // step but the last the next step's fragments are read between the MFMAs; the barrier follows the
  // step before the last, and the last step issues the copies of slice j + NST (spread evenly) and the
  // first fragments of slice j + 1 (in its second half).
  auto slice = [&]<bool REFILL, bool MORE>(int j) {
#pragma unroll
    for (int s = 0; s < ST; ++s) {
      u32x4(&cur)[NF] = f[s & 1];
      u32x4(&nxt)[NF] = f[(s + 1) & 1];
      const bool last = s == ST - 1;
#pragma unroll
      for (int k = 0; k < NS; ++k) {
        acc[k >> 2][k & 3] = mfma32<VAR>(cur[k >> 2], cur[TM + (k & 3)], acc[k >> 2][k & 3]);
        if (!last) {
          if (k < NF) nxt[k] = read1(j, s + 1, k);
        } else {
          if constexpr (REFILL)
#pragma unroll
            for (int i = 0; i < CPS; ++i)
              if (i * NS / CPS == k) copy1(j + NST, i);
          if constexpr (MORE)
#pragma unroll
            for (int r = 0; r < NF; ++r)
              if (NS / 2 + r * (NS / 2) / NF == k) nxt[r] = read1(j + 1, 0, r);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
      if (!last || MORE) lds_wait_all<NF>(nxt);
      if (s == ST - 2) {
        if (j + NST - 1 < L)
          wait_vm<YOUNG>();
        else
          wait_vm<0>();
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  };
  int j = 0;
  for (; j + NST < L; ++j) slice.template operator()<true, true>(j);
  for (; j + 1 < L; ++j) slice.template operator()<false, true>(j);
  slice.template operator()<false, false>(j);

#pragma unroll
  for (int n = 0; n < 4; ++n) {
    const int col = n0 + 128 * wn + 32 * n + ln;
    if (col >= N) continue;
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int m = m0 + (BM / 2) * wm + 32 * i + 8 * (e >> 2) + 4 * g + (e & 3);
        if (m < M) Y[(size_t)m * geo.ldy + col] = acc[i][n][e];
      }
  }
}

// ---- operand preparation --------------------------------------------------------------------------
// X fp16 [M, K] -> 16-bit [M, Kp] (fp16 as is, or rounded to bf16), zero columns K .. Kp - 1: for
// calls whose K is not a multiple of the slice or whose X is not 16-byte aligned.  One thread per
// output element.
__global__ __launch_bounds__(256) void k_pad_x16(const uint16_t* __restrict__ X, uint16_t* __restrict__ Y, int M,
                                                 int K, int Kp, int bf16) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (size_t)M * Kp) return;
  const size_t m = i / (size_t)Kp;
  const int k = (int)(i - m * (size_t)Kp);
  uint16_t v = 0;
  if (k < K) {
    v = X[m * (size_t)K + k];
    if (bf16) {
      const uint32_t u = __builtin_bit_cast(uint32_t, (float)__builtin_bit_cast(_Float16, v));  // exact
      v = (u & 0x7FFFFFFFu) > 0x7F800000u ? (uint16_t)((u >> 16) | 0x0040u)
                                          : (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
    }
  }
  Y[i] = v;
}

// Spreads R rows of K 16-bit values (contiguous) into rows of Kp (zero tail): one thread per output
// element, for weights whose K is not a multiple of the slice.
__global__ __launch_bounds__(256) void k_pad_rows16(const uint16_t* __restrict__ src, uint16_t* __restrict__ dst,
                                                    int R, int K, int Kp) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (size_t)R * Kp) return;
  const size_t r = i / (size_t)Kp;
  const int k = (int)(i - r * (size_t)Kp);
  dst[i] = k < K ? src[r * (size_t)K + k] : (uint16_t)0;
}

// fp16 -> bf16 (round to nearest even), 8 values a thread, X 16-byte aligned, M*K % 8 == 0; the same
// launch zeroes z4[0, nz4) (the tile counters of a K split).
__global__ __launch_bounds__(256) void k_x_to_bf16(const uint4* __restrict__ x, uint4* __restrict__ y, size_t n8,
                                                   float4* __restrict__ z4, size_t nz4) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  for (size_t k = i; k < nz4; k += (size_t)gridDim.x * 256) z4[k] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  if (i >= n8) return;
  const uint4 v = x[i];
  auto cv = [](uint32_t w) {
    uint32_t o = 0;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const uint32_t u = __builtin_bit_cast(uint32_t, (float)__builtin_bit_cast(_Float16, (uint16_t)(w >> (16 * h))));
      const uint32_t b = (u & 0x7FFFFFFFu) > 0x7F800000u ? ((u >> 16) | 0x0040u) : ((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
      o |= (b & 0xFFFFu) << (16 * h);
    }
    return o;
  };
  y[i] = make_uint4(cv(v.x), cv(v.y), cv(v.z), cv(v.w));
}

// Zeroes n4 float4s (the tile counters of a K split when no prepass runs).
__global__ __launch_bounds__(256) void k_zero16(float4* __restrict__ z4, size_t n4) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n4) z4[i] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
}

// ---- host side ------------------------------------------------------------------------------------

namespace {

inline int cdiv(int a, int b) { return (a + b - 1) / b; }

}  // namespace

int device_cus();

// Launch plan for M x N x K (K a multiple of 64): one or two launches over consecutive columns of 256
// weight rows.  A part runs 256-token tiles on the 4-wave kernel (k_gemm16q) or 128-token tiles on
// the 8-wave kernel (k_gemm16, 64-element slices); only a single 128-token part splits K (while its
// grid is below ~200 workgroups and each split keeps >= 8 slices).  The parts are chosen by rounds of
// workgroups times tile time, a 128-token tile costing 0.65 of a 256-token one (measured on MI355X:
// 63-65 us for one round of 128-token tiles at K = 4096, ~100 us a round of 256-token tiles): e.g.
// 2048 x 11008 runs one full round of 256-token tiles over 32 columns and the other 11 columns as
// one round of 128-token tiles (1.65 rounds of 256-token tile time, where a uniform grid takes 2).
struct G16Part {
  int bm, col0, ncols, mt, ntiles, splits, per;
};
struct G16Plan {
  int n;
  G16Part p[2];
};

G16Plan gemm16_plan(int M, int N, int K, int cus, int max_splits = 64) {
  const int nt = cdiv(N, kBN), nsl = K / 64;
  const int m256 = cdiv(M, 256), m128 = cdiv(M, 128);
  auto rounds = [&](int tiles) { return (double)cdiv(tiles, cus); };
  constexpr double kT128 = 0.65;
  G16Plan pl{};
  pl.n = 1;
  // uniform 128-token tiles, K split while the grid is small
  G16Part q{128, 0, nt, m128, nt * m128, 1, nsl};
  while (q.ntiles * q.splits < 200 * cus / 256 && nsl / (q.splits * 2) >= 8 && q.splits * 2 <= max_splits)
    q.splits *= 2;
  q.per = cdiv(nsl, q.splits);
  q.splits = cdiv(nsl, q.per);
  pl.p[0] = q;
  double best = rounds(q.ntiles * q.splits) * kT128 / q.splits + (q.splits > 1 ? 0.02 : 0.0);
  // uniform 256-token tiles
  if (const double c = rounds(nt * m256); c < best - 1e-9) {
    best = c;
    pl.p[0] = G16Part{256, 0, nt, m256, nt * m256, 1, nsl};
  }
  // 256-token tiles on the first c1 columns, 128-token tiles on the rest
  for (int c1 = 1; c1 < nt; ++c1) {
    const double c = rounds(c1 * m256) + rounds((nt - c1) * m128) * kT128 + 0.03;
    if (c < best - 1e-9) {
      best = c;
      pl.n = 2;
      pl.p[0] = G16Part{256, 0, c1, m256, c1 * m256, 1, nsl};
      pl.p[1] = G16Part{128, c1, nt - c1, m128, (nt - c1) * m128, 1, nsl};
    }
  }
  return pl;
}

// Bytes of a plan's K-split workspace (partial tiles, then the counters, whose size *cbytes is
// 256-byte aligned); 0 without a split.
size_t gemm16_split_bytes(const G16Plan& pl, size_t* cbytes) {
  const G16Part& p = pl.p[0];
  if (pl.n != 1 || p.splits <= 1) {
    *cbytes = 0;
    return 0;
  }
  *cbytes = ((size_t)p.ntiles * 4 + 255) & ~(size_t)255;
  return (size_t)p.ntiles * p.splits * p.bm * kBN * 4 + *cbytes;
}

// Launches the GEMM of plan pl; split_ws: gemm16_split_bytes(pl) bytes, counters (its last cbytes)
// zero, or scnt: zeroed counters to use in place of those (a stream's block).  X and B rows are K
// 16-bit values (K % 64 == 0), both 16-byte aligned.
bool launch_gemm16(const G16Plan& pl, float* out, int ldy, const uint16_t* X, const uint16_t* B, int M, int N, int K,
                   bool bf16, void* split_ws, hipStream_t s, uint32_t* scnt = nullptr) {
  size_t cb = 0;
  const size_t sb = gemm16_split_bytes(pl, &cb);
  if (sb && !split_ws) return false;
  for (int i = 0; i < pl.n; ++i) {
    const G16Part& p = pl.p[i];
    const int r0 = p.col0 * kBN, nr = std::min(N - r0, p.ncols * kBN);
    if (nr <= 0) continue;
    Geo geo{M, nr, K, ldy, p.mt, p.per, sb ? static_cast<float*>(split_ws) : nullptr,
            !sb ? nullptr : scnt ? scnt : reinterpret_cast<uint32_t*>(static_cast<uint8_t*>(split_ws) + sb - cb)};
    const uint16_t* Bp = B + (size_t)r0 * K;
    float* op = out + r0;
    const dim3 grid((unsigned)p.ntiles, 1, (unsigned)p.splits);
    if (p.bm == 256) {
      if (bf16)
        k_gemm16q<VAR_BF16, 256, 64, 2><<<grid, 256, 0, s>>>(X, Bp, op, geo);
      else
        k_gemm16q<VAR_F16, 256, 64, 2><<<grid, 256, 0, s>>>(X, Bp, op, geo);
    } else {
      if (bf16)
        k_gemm16<VAR_BF16, 128, 64><<<grid, 512, 0, s>>>(X, Bp, op, geo);
      else
        k_gemm16<VAR_F16, 128, 64><<<grid, 512, 0, s>>>(X, Bp, op, geo);
    }
  }
  return true;
}

void launch_zero16(void* p, size_t bytes, hipStream_t s) {
  const size_t n4 = bytes / 16;
  if (n4) k_zero16<<<(unsigned)((n4 + 255) / 256), 256, 0, s>>>(static_cast<float4*>(p), n4);
}

bool launch_dequant16(uint32_t t, const void* src, uint16_t* dst, size_t n, bool bf16, hipStream_t s);
bool launch_dequant16_bf16_x(uint32_t t, const void* src, uint16_t* dst, size_t n, const uint16_t* x, uint16_t* xo,
                             size_t n8, hipStream_t s);
void* gemm_temp_alloc(size_t bytes, hipStream_t s);
void gemm_temp_free(void* p, hipStream_t s);
uint32_t* gemm_stream_counters(size_t n, hipStream_t s);

// Plain 16-bit GEMM entry (qvx_gemm16): out [M, N] = X [M, K] . B [N, K]^T, both operands bf16 or fp16.
// Temporaries (padded copies when K % 64 != 0 or an operand is not 16-byte aligned, a K split's
// partial tiles) come from the library's pool.  Returns a QVX status.
int launch_gemm16_entry(float* out, const uint16_t* X, const uint16_t* B, int M, int N, int K, bool bf16,
                        hipStream_t s) {
  const int Kp = (K + 63) & ~63;
  if ((size_t)256 * (size_t)Kp * 2u >= (1u << 31)) return -7;
  const bool padx = Kp != K || (reinterpret_cast<uintptr_t>(X) & 15u);
  const bool padb = Kp != K || (reinterpret_cast<uintptr_t>(B) & 15u);
  const G16Plan p = gemm16_plan(M, N, Kp, device_cus());
  size_t cb = 0;
  const size_t sb = gemm16_split_bytes(p, &cb);
  const size_t xb = padx ? (((size_t)M * Kp * 2u + 255) & ~(size_t)255) : 0;
  const size_t bb = padb ? (((size_t)N * Kp * 2u + 255) & ~(size_t)255) : 0;
  uint8_t* tmp = nullptr;
  if (xb + bb + sb) {
    tmp = static_cast<uint8_t*>(gemm_temp_alloc(xb + bb + sb, s));
    if (!tmp) return -5;
  }
  const uint16_t* Xg = X;
  const uint16_t* Bg = B;
  if (padx) {
    const size_t n = (size_t)M * Kp;
    k_pad_rows16<<<(unsigned)((n + 255) / 256), 256, 0, s>>>(X, reinterpret_cast<uint16_t*>(tmp), M, K, Kp);
    Xg = reinterpret_cast<const uint16_t*>(tmp);
  }
  if (padb) {
    const size_t n = (size_t)N * Kp;
    k_pad_rows16<<<(unsigned)((n + 255) / 256), 256, 0, s>>>(B, reinterpret_cast<uint16_t*>(tmp + xb), N, K, Kp);
    Bg = reinterpret_cast<const uint16_t*>(tmp + xb);
  }
  // the K split's counters: the stream's zeroed block, else the temporary's, cleared here
  uint32_t* scnt = sb ? gemm_stream_counters((size_t)p.p[0].ntiles, s) : nullptr;
  if (sb && !scnt) launch_zero16(tmp + xb + bb + sb - cb, cb, s);
  const bool ok = launch_gemm16(p, out, N, Xg, Bg, M, N, Kp, bf16, sb ? tmp + xb + bb : nullptr, s, scnt);
  if (tmp) gemm_temp_free(tmp, s);
  return ok ? 0 : -5;
}

// Prefill GEMM of a weight dequantised into 16 bits (every type qvx_qgemm_f16 takes that has no
// raw-block kernel): X fp16 [M, cols] -> 16-bit operand (bf16 variant: rounded; K padded to 64 or X
// unaligned: a padded copy), then per panel of P weight rows: the rows dequantised into a 16-bit
// buffer (the reference's value rounded once), and k_gemm16 writes output columns r0 .. r0 + P - 1.
// Temporaries come from the caller's region [ws, ws + ws_cap) when ws is set (the no-allocation
// entry point: panels are sized to fit it, QVX_E_RANGE when not even one 256-row panel does), else
// from the library's pool in one piece (one panel).  Returns a QVX status.
int launch_qgemm_via16(float* out, const void* w, uint32_t t, const uint16_t* X, int M, int rows, int cols, bool bf16,
                       hipStream_t s, void* ws, size_t ws_cap) {
  const TypeInfo* ti = type_info(t);
  if (!ti || !can_dequantize(t)) return -1;
  const size_t row_bytes = (size_t)(cols / (int)ti->block) * ti->bytes;
  const int Kp = (cols + 63) & ~63;
  if ((size_t)256 * (size_t)Kp * 2u >= (1u << 31)) return -7;
  const bool padk = Kp != cols;
  const bool padx = padk || (reinterpret_cast<uintptr_t>(X) & 15u);
  const bool xcopy = padx || bf16;
  const size_t xb = xcopy ? (((size_t)M * Kp * 2u + 255) & ~(size_t)255) : 0;
  const int cus = device_cus();
  // Bytes a panel of P rows needs: its 16-bit weight (plus the unpadded dequant when K is padded)
  // and its plan's K-split workspace (at most ms splits).
  auto panel_bytes = [&](int P, int ms, G16Plan* pp) {
    const G16Plan p = gemm16_plan(M, P, Kp, cus, ms);
    if (pp) *pp = p;
    size_t cb = 0;
    const size_t wb = ((size_t)P * Kp * 2u + 255) & ~(size_t)255;
    const size_t ub = padk ? (((size_t)P * cols * 2u + 255) & ~(size_t)255) : 0;
    return wb + ub + gemm16_split_bytes(p, &cb);
  };
  // Panel rows and split cap: one panel from the pool; in a caller's region the largest panel (whole,
  // then halves rounded to 256 rows, down to 256) that fits with some split count, fewer splits
  // before fewer rows.
  int P = rows, ms = 64;
  if (ws) {
    bool fit = false;
    for (int cand = rows;; cand = std::max(256, ((cand / 2) + 255) & ~255)) {
      for (int m = 64; m >= 1 && !fit; m /= 2)
        if (xb + panel_bytes(cand, m, nullptr) <= ws_cap) {
          P = cand;
          ms = m;
          fit = true;
        }
      if (fit || cand <= 256) break;
    }
    if (!fit) return -7;
  }
  uint8_t* tmp = static_cast<uint8_t*>(ws ? ws : gemm_temp_alloc(xb + panel_bytes(P, ms, nullptr), s));
  if (!tmp) return -5;
  const uint16_t* Xg = X;
  uint16_t* xc = reinterpret_cast<uint16_t*>(tmp);
  // bf16 X without padding: rounded in the first panel's dequantisation launch when the wide
  // dequantiser takes that panel (one memory-bound launch instead of two), else by its own prepass
  bool x_pending = false;
  const size_t xn8 = (size_t)M * cols / 8;
  auto x_prepass = [&]() {
    k_x_to_bf16<<<(unsigned)((xn8 + 255) / 256), 256, 0, s>>>(reinterpret_cast<const uint4*>(X),
                                                               reinterpret_cast<uint4*>(xc), xn8, nullptr, 0);
  };
  if (padx) {
    const size_t n = (size_t)M * Kp;
    k_pad_x16<<<(unsigned)((n + 255) / 256), 256, 0, s>>>(X, xc, M, cols, Kp, bf16 ? 1 : 0);
    Xg = xc;
  } else if (bf16) {
    x_pending = true;
    Xg = xc;
  }
  uint16_t* wd = reinterpret_cast<uint16_t*>(tmp + xb);
  int rc = 0;
  for (int r0 = 0; r0 < rows && rc == 0; r0 += P) {
    const int pr = std::min(P, rows - r0);
    G16Plan plan;
    size_t cb = 0;
    (void)panel_bytes(pr, ms, &plan);
    const size_t wb = ((size_t)pr * Kp * 2u + 255) & ~(size_t)255;
    const size_t ub = padk ? (((size_t)pr * cols * 2u + 255) & ~(size_t)255) : 0;
    const size_t sb = gemm16_split_bytes(plan, &cb);
    const uint8_t* wsrc = static_cast<const uint8_t*>(w) + (size_t)r0 * row_bytes;
    if (padk) {
      uint16_t* u = reinterpret_cast<uint16_t*>(tmp + xb + wb);
      if (!launch_dequant16(t, wsrc, u, (size_t)pr * cols, bf16, s)) {
        rc = -1;
        break;
      }
      const size_t n = (size_t)pr * Kp;
      k_pad_rows16<<<(unsigned)((n + 255) / 256), 256, 0, s>>>(u, wd, pr, cols, Kp);
    } else if (x_pending && launch_dequant16_bf16_x(t, wsrc, wd, (size_t)pr * cols, X, xc, xn8, s)) {
      x_pending = false;
    } else {
      if (x_pending) {
        x_prepass();
        x_pending = false;
      }
      if (!launch_dequant16(t, wsrc, wd, (size_t)pr * cols, bf16, s)) {
        rc = -1;
        break;
      }
    }
    uint8_t* split_ws = sb ? tmp + xb + wb + ub : nullptr;
    // the K split's counters: the stream's zeroed block for calls that may allocate, else the
    // region's, cleared here
    uint32_t* scnt = sb && !ws ? gemm_stream_counters((size_t)plan.p[0].ntiles, s) : nullptr;
    if (sb && !scnt) launch_zero16(split_ws + sb - cb, cb, s);
    if (!launch_gemm16(plan, out + r0, rows, Xg, wd, M, pr, Kp, bf16, split_ws, s, scnt)) rc = -5;
  }
  if (!ws) gemm_temp_free(tmp, s);
  return rc;
}

}  // namespace qvx
