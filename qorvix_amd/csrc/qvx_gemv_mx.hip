// qvx_gemv_mx.hip -- matrix-core GEMV for Q4_K on gfx950 (M = 1..8 vectors per launch).
//
// out[v, r] = sum_k dequant(W)[r, k] * X[v, k]   (the reference's qmatmul / qmatmulN,
// runtime/src/qmatmul.cpp:28-115) with the integer arithmetic of the VALU GEMV (qvx_gemv.hip):
// activations in 15-bit fixed point per 64-element group (q = 128 qh + ql, two signed bytes),
// quant codes as signed bytes (low nibbles n, high nibbles 16 (n - 8)), exact int32 dot products,
// one affine fold per (row, group).  Only the dot products move to v_mfma_i32_16x16x64_i8.
//
// MFMA mapping for one tile = 16 weight rows x one super-block (256 columns), 4 MFMAs:
//  * B (16 columns = weight rows j, K = 64): lane (j, g) (j = lane%16, g = lane/16) supplies for
//    MFMA m the 16 codes of bytes 8m..8m+7 of row j's scale group g (qs bytes 32g..32g+31): the 8
//    low nibbles (elements 64g + 8m + 0..7, sub-block 2g) and the 8 high nibbles (elements
//    64g + 32 + 8m + 0..7, sub-block 2g+1).
//  * A (16 rows = (group c, part p), row 4c + p): lane (4c + p, g) is nonzero only for g == c and
//    holds, at the same K positions, qh (p = 0) or ql (p = 1) of the low-nibble elements with zeros
//    at the high-nibble positions, or zeros and qh (p = 2) / ql (p = 3) of the high-nibble elements.
//    Only the nonzero halves are built, once per workgroup, in LDS: 8 bytes per (group, part, m),
//    512 bytes per (vector, super-block); the lane reads its part's 32 bytes (all four m) and makes
//    the zero half of each operand, and the whole operand of a lane with g != c, with masks.
//  * After the 4 MFMAs the accumulator of lane (j, c) holds rows 4c..4c+3 of column j, i.e. the
//    four partial sums (lo.qh, lo.ql, hi.qh, hi.ql) of row j over group c: the lane applies the
//    group's scale/min fold exactly as the VALU kernel does.  K positions are matched between A
//    and B lane by lane and register by register, so the product does not depend on how the
//    instruction orders K inside a lane group.
//
// Data movement: each wave owns a ring of NB = 2 LDS stages.  A tile's 2304 bytes (16 rows x 144,
// rows 144 bytes apart in LDS: conflict-free for the 16-lane quarter reads) are copied by three
// buffer_load ... lds with all 64 lanes active: two 16-byte copies (lane l of copy k fills LDS
// bytes 1024k + 16l..+15, i.e. row q/9, 16-byte chunk q%9 for q = 64k + l) and one 4-byte copy
// for the last 256 bytes (lane l fills byte p = 2048 + 4l: row p/144, column p%144).  With no lane
// condition on any copy there is no branch for the compiler to wait across.  (A 12-byte copy would
// not do: it places each lane's 12 bytes at a 16-byte pitch in LDS.)  The super-block offset is
// the scalar soffset.  The prologue fills both stages; a stage is refilled with the tile two
// super-blocks on as soon as its contents are in registers, so two tiles are in flight while one
// is folded.  The wave waits for a tile with s_waitcnt vmcnt (the copies are its only vector
// memory operations in the loop) and reads it back in MFMA order, through inline asm (see
// lds_read16).  Waves with activation conversion tasks load and convert before their first copy;
// the others copy at once.

// Work: workgroup b owns rows [rb, rb + cnt) (cnt <= 16 TQ); wave w = kq * TQ + tq takes tile tq
// and super-blocks [kq nsb / KQ, (kq + 1) nsb / KQ).  Per-lane partials are summed over the four
// groups with permlane swaps and over the KQ waves of a tile in wave order through LDS, so every
// output's arithmetic is fixed: one vector's result does not depend on the other vectors of the
// launch, and qvx_qmatmul_n stays bit-identical to qvx_qmatmul per vector.
#include <algorithm>

#include "qvx_common.hpp"
#include "qvx_gemv_valu.hpp"
#include "qvx_norm.hpp"

namespace qvx {

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef short short2_t __attribute__((ext_vector_type(2)));
#define QVX_LDS __attribute__((address_space(3)))

constexpr int kSB = 144;          // Q4_K super-block bytes
constexpr int kTileBytes = 2304;  // 16 rows x one super-block
constexpr int kFragBytes = 512;  // A fragment halves of one (vector, super-block): [group][part][m] x 8 bytes
constexpr uint32_t kRsrcWord3 = 0x00020000u;  // raw buffer, 32-bit data (gfx9)

struct MxGeo {
  int nsb;        // super-blocks per row
  int base, rem;  // workgroup b owns base + unit (b < rem) rows starting at b*base + unit min(b, rem)
  int unit;       // rows come in whole units: 1, or 32 (a fused SwiGLU launch: 16 gate + 16 up rows)
  int TQ, KQ;     // tiles per workgroup, K splits; TQ * KQ = 16 waves
  uint32_t row_bytes;
};

// LDS: dynamic [fragments: NV*nsb*512][meta: NV*nsb*4 groups*16], a static tile ring
// [16 waves][NB][2304] and the partial sums [16 waves][NV][16] floats.
__host__ __device__ inline size_t mx_frag_bytes(int nv, int nsb) { return (size_t)nv * nsb * kFragBytes; }
__host__ __device__ inline size_t mx_meta_bytes(int nv, int nsb) { return (size_t)nv * nsb * 4 * 16; }
__host__ __device__ inline size_t mx_dyn_bytes(int nv, int nsb) { return mx_frag_bytes(nv, nsb) + mx_meta_bytes(nv, nsb); }
__host__ __device__ inline size_t mx_lds_bytes(int nv, int nsb, int nb) {
  return mx_dyn_bytes(nv, nsb) + (size_t)16 * nb * kTileBytes + (size_t)16 * nv * 16 * 4;
}

template <int CTRL>
__device__ inline float dppf(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
template <int CTRL>
__device__ inline int dppi(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}
constexpr int kXor1 = 0xB1, kXor2 = 0x4E, kHalfMirror = 0x141;

__device__ inline uint32_t hi_codes(uint32_t w) { return (w & 0xF0F0F0F0u) ^ 0x80808080u; }

// s_waitcnt vmcnt(N) with the other counters left alone (gfx9 encoding).
template <int N>
__device__ inline void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// LDS read of 16 bytes the compiler does not track.  The main loop reads LDS only through this:
// the compiler cannot tell these reads from the ring that the in-flight copies write and would
// otherwise wait for every copy (vmcnt(0)) before each read.  The copies are synchronised
// explicitly with s_waitcnt vmcnt, and lds_wait() (which takes the results as operands, so no use
// can move above it) waits for the reads.
template <int OFF = 0>
__device__ inline u32x4 lds_read16(uint32_t addr) {
  u32x4 r;
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "i"(OFF) : "memory");
  return r;
}
__device__ inline void lds_wait(u32x4& a, u32x4& b, u32x4& c) {
  asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(a), "+v"(b), "+v"(c)::"memory");
}

// LDS write the compiler does not track, for the same reason: were a copy of this wave in flight
// it would wait for all of them (vmcnt(0)) before an LDS store it emits, so the fragment stores do
// not depend on the code order.  They never overlap the copy ring, and the lgkmcnt(0) before the
// barrier that follows them orders them for the readers.
__device__ inline uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(QVX_LDS const uint8_t*)p;
}
__device__ inline void lds_write8(uint32_t addr, uint32_t lo, uint32_t hi) {
  typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
  const u32x2 v = {lo, hi};
  asm volatile("ds_write_b64 %0, %1" ::"v"(addr), "v"(v) : "memory");
}

// ---- activations -> A fragments ---------------------------------------------------------------
// Task t (per vector nsb*32 tasks) = 8 elements: part p = t%8 of group (s, g) = (t/8)/4, (t/8)%4,
// elements 256 s + 64 g + 8 p + 0..7; the 8 tasks of a group are 8 aligned lanes.
template <int NV>
__device__ inline int task_vec(int t, int per) {
  int v = 0;
#pragma unroll
  for (int i = 1; i < NV; ++i) v += t >= i * per ? 1 : 0;
  return v;
}

// The 15-bit fixed-point form of one task's 8 activations: qh / ql bytes (elements 0..3 in h0 / l0,
// 4..7 in h1 / l1), the group's step sx (NaN when the group holds a non-finite value) and the sum
// of q over the task's half of the group.  Every lane of the wave calls it (DPP across the 8 tasks
// of a group).  Both GEMV layouts convert through this one function, so their arithmetic agrees.
struct XQ8 {
  uint32_t h0, h1, l0, l1;
  float sx;
  int sq;
};
__device__ inline XQ8 mx_quantize(const float4 x0, const float4 x1) {
  float a = fmaxf(fmaxf(fmaxf(fabsf(x0.x), fabsf(x0.y)), fmaxf(fabsf(x0.z), fabsf(x0.w))),
                  fmaxf(fmaxf(fabsf(x1.x), fabsf(x1.y)), fmaxf(fabsf(x1.z), fabsf(x1.w))));
  // 0 when the eight elements are finite, NaN otherwise (x * 0 is NaN for +-Inf and NaN)
  float z = __builtin_fmaf(x0.x, 0.0f, __builtin_fmaf(x0.y, 0.0f, __builtin_fmaf(x0.z, 0.0f, x0.w * 0.0f)));
  z = __builtin_fmaf(x1.x, 0.0f, __builtin_fmaf(x1.y, 0.0f, __builtin_fmaf(x1.z, 0.0f, __builtin_fmaf(x1.w, 0.0f, z))));
  a = fmaxf(a, dppf<kXor1>(a));
  a = fmaxf(a, dppf<kXor2>(a));
  a = fmaxf(a, dppf<kHalfMirror>(a));
  z += dppf<kXor1>(z);
  z += dppf<kXor2>(z);
  z += dppf<kHalfMirror>(z);
  // k = 16383 / (32767 amax): v_cvt_pknorm_i16_f32 returns rn(clamp(y, -1, 1) * 32767)
  const float k = (a > 0.0f && a <= 3.402823466e38f) ? __builtin_amdgcn_rcpf(a) * (16383.0f / 32767.0f) : 0.0f;
  const uint32_t p[4] = {
      __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pknorm_i16(x0.x * k, x0.y * k)),
      __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pknorm_i16(x0.z * k, x0.w * k)),
      __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pknorm_i16(x1.x * k, x1.y * k)),
      __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pknorm_i16(x1.z * k, x1.w * k))};
  uint32_t hs[4], ls[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    hs[i] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(short2_t, p[i]) >> (short)7);  // q >> 7 per half
    ls[i] = p[i] & 0x007F007Fu;                                                              // q & 127 per half
  }
  const short2_t ones = {1, 1};
  int sq = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) sq = __builtin_amdgcn_sdot2(__builtin_bit_cast(short2_t, p[i]), ones, sq, false);
  sq += dppi<kXor1>(sq);
  sq += dppi<kXor2>(sq);  // sum of q over the 32 elements of this task's half of the group
  XQ8 r;
  r.h0 = __builtin_amdgcn_perm(hs[1], hs[0], 0x06040200u);
  r.h1 = __builtin_amdgcn_perm(hs[3], hs[2], 0x06040200u);
  r.l0 = __builtin_amdgcn_perm(ls[1], ls[0], 0x06040200u);
  r.l1 = __builtin_amdgcn_perm(ls[3], ls[2], 0x06040200u);
  r.sx = a * (1.0f / 16383.0f) + z;
  r.sq = sq;
  return r;
}

__device__ inline void mx_convert(const float4 x0, const float4 x1, int v, int sg, int part, bool store,
                                  uint8_t* frag, float* meta, int nsb) {
  const XQ8 q = mx_quantize(x0, x1);
  if (store) {
    const int g = sg & 3, s = sg >> 2, hi = part >> 2, m = part & 3;
    const uint32_t f = lds_addr(frag) + (uint32_t)((v * nsb + s) * kFragBytes + g * 128 + 2 * hi * 32 + m * 8);
    lds_write8(f, q.h0, q.h1);       // part 2hi: qh
    lds_write8(f + 32, q.l0, q.l1);  // part 2hi + 1: ql
    const uint32_t mt = lds_addr(meta) + (uint32_t)(((v * nsb + s) * 4 + g) * 16);  // [sx, Qa, Qb, 128 Qb as int]
    if (part == 0) lds_write8(mt, __builtin_bit_cast(uint32_t, q.sx), __builtin_bit_cast(uint32_t, (float)q.sq));
    if (part == 4) lds_write8(mt + 8, __builtin_bit_cast(uint32_t, (float)q.sq), (uint32_t)(128 * q.sq));
  }
}

// RMSNorm folded into the conversion (the batched form shares it): each wave's 64 tasks of round k
// are 512 consecutive elements of one vector (cols % 512 == 0); their sum of squares goes to LDS as
// chunk (v, c), and after a barrier every task scales its 8 elements by its vector's factor.  Tasks
// past ntask (clamped duplicates) add nothing.
template <int TPT>
__device__ inline void mx_norm(float4 (&xa)[TPT], float4 (&xb)[TPT], const float4 (&wa)[TPT],
                               const float4 (&wb)[TPT], int tid, int per, int ntask, int cols, float eps,
                               float* sqp) {
  const int wave = tid >> 6, lane = tid & 63;
  const uint32_t sq_base = lds_addr(sqp);
#pragma unroll
  for (int k = 0; k < TPT; ++k) {
    const int tw = 1024 * k + 64 * wave;  // the wave's first task (uniform)
    if (tw < ntask) {
      const float s = wave_sum64(tid + 1024 * k < ntask ? norm_sq8(xa[k], xb[k]) : 0.0f);
      const int v = tw / per, c = (tw - v * per) >> 6;
      if (lane == 0) norm_store(sq_base + 4u * (uint32_t)(v * kNormMaxChunks + c), s);
    }
  }
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
  __builtin_amdgcn_s_barrier();
#pragma unroll
  for (int k = 0; k < TPT; ++k) {
    if (1024 * k + 64 * wave < ntask) {
      const int t = min(tid + 1024 * k, ntask - 1), v = t / per;
      const float scale = norm_scale(sq_base + 4u * (uint32_t)(v * kNormMaxChunks), per >> 6, cols, eps);
      norm_apply(xa[k], xb[k], scale, wa[k], wb[k]);
    }
  }
}

// Final outputs from the per-wave partials red[tq][kq][v][16] (every K-split wave of a tile, in wave
// order): plain rows, or with EPI_SWIGLU silu(gate) * up of each (gate tile 2p, up tile 2p + 1)
// pair, written at output row (rb + 32 p) / 2 + r of the rows / 2 a vector has.
template <int EPI>
__device__ inline void mx_store(const float* red, float* Y, int nv, int rows, int rb, int cnt, int TQ, int KQ,
                                int tid) {
  if constexpr ((EPI & EPI_SWIGLU) != 0) {
    const int half = rows >> 1;
    for (int o = tid; o < (TQ >> 1) * nv * 16; o += 1024) {
      const int p = o / (nv * 16), v = (o >> 4) % nv, r = o & 15;
      if (32 * p < cnt) {
        float g = 0.0f, u = 0.0f;
        for (int k = 0; k < KQ; ++k) {
          g += red[((2 * p * KQ + k) * nv + v) * 16 + r];
          u += red[(((2 * p + 1) * KQ + k) * nv + v) * 16 + r];
        }
        Y[(size_t)v * half + (rb >> 1) + 16 * p + r] = silu_mul(g, u);
      }
    }
  } else {
    for (int o = tid; o < TQ * nv * 16; o += 1024) {
      const int t = o / (nv * 16), v = (o >> 4) % nv, r = o & 15;
      const int row = 16 * t + r;
      if (row < cnt) {
        float sum = 0.0f;
        for (int k = 0; k < KQ; ++k) sum += red[((t * KQ + k) * nv + v) * 16 + r];
        Y[(size_t)v * rows + rb + row] = sum;
      }
    }
  }
}

// Step u of a K-split wave -> super-block.  Even waves of a split walk their range backwards, odd
// waves forwards: a 128-byte line that straddles two waves' ranges (super-blocks are 144 bytes, so
// most split points fall inside a line) is then requested by both waves at the same moment -- at
// the start of both walks or at the end of both -- and fetched from HBM once, instead of once at
// the start of one walk and again, long evicted from L2, at the end of the other.  All three forms
// (one-vector, batched, long-row batched) walk the same order, so their folds stay identical.
struct SbOrder {
  int base, step;
  __device__ SbOrder(int kq, int KQ, int s0, int s1)
      : base(KQ > 1 && !(kq & 1) ? s1 - 1 : s0), step(KQ > 1 && !(kq & 1) ? -1 : 1) {}
  __device__ int operator()(int u) const { return base + step * u; }
};

// Copy a tile (16 rows of this wave, super-block s) into an LDS stage: 2 x 1024 + 256 bytes.
__device__ inline void mx_issue(__amdgpu_buffer_rsrc_t rsrc, const uint32_t (&off)[3], int s, QVX_LDS uint8_t* st) {
  const uint32_t so = (uint32_t)s * kSB;
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, st, 16, off[0], so, 0, 0);
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, st + 1024, 16, off[1], so, 0, 0);
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, st + 2048, 4, off[2], so, 0, 0);
}

// EPI: EPI_NORM takes rmsnorm(x, NW, eps) as the activations (folded into the conversion: the
// workgroup's tasks cover every element of its vectors); EPI_SWIGLU takes rows interleaved in
// 16-row (gate, up) groups (geo.unit = 32) and writes silu(gate) * up, rows / 2 outputs a vector.
// The kernel's body for workgroup b (the standalone kernel passes blockIdx.x, a grouped launch its
// own block numbering).
template <int NV, int NB, int TPT, int EPI>
__device__ __forceinline__ void gemv_mx_body(const uint8_t* __restrict__ W, const float* __restrict__ X,
                                             float* __restrict__ Y, int rows, int cols, const MxGeo& geo,
                                             const float* __restrict__ NW, float eps, int b) {
  static_assert(NB >= 2 && NB <= 4, "the tile wait below covers up to 3 tiles ahead");
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  __shared__ __attribute__((aligned(16))) uint8_t ring[16 * NB * kTileBytes];
  __shared__ float red[16 * NV * 16];  // per-wave partial sums [tq][kq][v][16]
  __shared__ __attribute__((aligned(16))) float sqp[(EPI & EPI_NORM) ? NV * kNormMaxChunks : 4];  // chunk sums
  const int nsb = geo.nsb, TQ = geo.TQ, KQ = geo.KQ;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: scalar offsets, M0
  uint8_t* frag = lds;
  float* meta = reinterpret_cast<float*>(lds + mx_frag_bytes(NV, nsb));
  QVX_LDS uint8_t* stage = (QVX_LDS uint8_t*)(ring + wave * NB * kTileBytes);

  const int rb = b * geo.base + geo.unit * min(b, geo.rem), cnt = geo.base + (b < geo.rem ? geo.unit : 0);
  const int tq = wave % TQ, kq = wave / TQ;
  const int s0 = kq * nsb / KQ, s1 = (kq + 1) * nsb / KQ, nu = s1 - s0;
  const SbOrder order(kq, KQ, s0, s1);

  // 1. activation loads (waves that hold conversion tasks), then 2. the prologue tile copies, then
  // 3. the conversion into A fragments.  The activation loads go first: a wave's vector memory
  // instructions stall at issue once the CU's queue of outstanding requests is full, and the CU
  // returns data in request order, so activation loads behind tile copies would wait out the HBM
  // latency and hold the fragment barrier back.  The copies go before the conversion so that the
  // tiles are in flight while it runs (one launch of 4096 -> 14336 3 % faster, of 4096 -> 4096 9 %).
  // Waves without tasks go straight to their copies.  Every round's loads go out before the first
  // conversion (see the batched form).
  const int per = nsb * 32, ntask = NV * per;
  float4 xa[TPT], xb[TPT], wa[TPT], wb[TPT];
#pragma unroll
  for (int k = 0; k < TPT; ++k) {
    if (1024 * k + 64 * wave < ntask) {
      const int t = min(tid + 1024 * k, ntask - 1), v = task_vec<NV>(t, per), r = t - v * per;
      const float4* src = reinterpret_cast<const float4*>(X + (size_t)v * cols + 8 * r);
      xa[k] = src[0];
      xb[k] = src[1];
    }
  }
  // 2. prologue copies into all NB stages (tiles of super-blocks s0.., repeating the wave's last one
  // when it has fewer than NB, so the count is fixed; rows past cnt read as zeros)
  const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(W + (size_t)rb * geo.row_bytes), (short)0, (int)((uint32_t)cnt * geo.row_bytes), (int)kRsrcWord3);
  uint32_t off[3];
#pragma unroll
  for (int k = 0; k < 3; ++k) {
    // LDS byte of this lane's chunk in the tile, then its row and column (chunks never cross rows).
    const uint32_t p = k < 2 ? (uint32_t)(1024 * k + 16 * lane) : (uint32_t)(2048 + 4 * lane);
    const uint32_t r = p / (uint32_t)kSB, c = p - (uint32_t)kSB * r;
    off[k] = __umul24(16u * (uint32_t)tq + r, geo.row_bytes) + c;
  }
#pragma unroll
  for (int u = 0; u < NB; ++u) mx_issue(rsrc, off, nu > 0 ? order(min(u, nu - 1)) : s0, stage + u * kTileBytes);
  // the norm weights are needed only after the sums of squares: behind the copies, so the tiles'
  // requests are not queued behind them (a q|k launch with the norm 6.57 -> 6.28 us)
  if constexpr ((EPI & EPI_NORM) != 0) {
#pragma unroll
    for (int k = 0; k < TPT; ++k) {
      if (1024 * k + 64 * wave < ntask) {
        const int t = min(tid + 1024 * k, ntask - 1), r = t - task_vec<NV>(t, per) * per;
        wa[k] = reinterpret_cast<const float4*>(NW + 8 * r)[0];
        wb[k] = reinterpret_cast<const float4*>(NW + 8 * r)[1];
      }
    }
  }

  if constexpr ((EPI & EPI_NORM) != 0) mx_norm<TPT>(xa, xb, wa, wb, tid, per, ntask, cols, eps, sqp);
#pragma unroll
  for (int k = 0; k < TPT; ++k) {
    if (1024 * k + 64 * wave < ntask) {
      const int t0 = tid + 1024 * k, t = min(t0, ntask - 1), v = task_vec<NV>(t, per), r = t - v * per;
      mx_convert(xa[k], xb[k], v, r >> 3, r & 7, t0 < ntask, frag, meta, nsb);
    }
  }

  // Barrier for the fragments only: wait for this wave's LDS writes, not for the tile copies in
  // flight (__syncthreads would wait for those too).
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
  __builtin_amdgcn_s_barrier();

  // 4. tiles
  const int j = lane & 15, g = lane >> 4;  // B column (tile row) / K block = group; A row = j
  const uint32_t b_hd = kSB * j, b_q = kSB * j + 16 + 32 * g;
  const bool aon = (j >> 2) == g;
  // A operand: this lane's part p = j & 3 of group g (32 bytes, m = 0..3), in the low half of the
  // operand for p < 2 and the high half for p >= 2, all zero unless g == j / 4
  const uint32_t a_rel = (uint32_t)(g * 128 + (j & 3) * 32);
  const uint32_t mlo = aon && (j & 3) < 2 ? ~0u : 0u, mhi = aon && (j & 3) >= 2 ? ~0u : 0u;
  const uint32_t frag_base = (uint32_t)(uintptr_t)(QVX_LDS uint8_t*)frag;
  const uint32_t meta_base = (uint32_t)(uintptr_t)(QVX_LDS uint8_t*)meta + 16u * g;
  const uint32_t stage_base = (uint32_t)(uintptr_t)stage;
  // fold constants of group g (the VALU kernel's Q4_K scale unpacking)
  const uint32_t jj = 2u * (uint32_t)(g & 1);
  const uint32_t sel1 = jj | (jj + 1) << 8 | (jj + 4) << 16 | (jj + 5) << 24;
  const uint32_t sel2 = jj | (jj + 1) << 8 | jj << 16 | (jj + 1) << 24;
  const bool up = g >= 2;
  const uint32_t m1 = up ? 0u : 0x3F3F3F3Fu, m2 = up ? 0x30303030u : 0u, m3 = up ? 0x00000F0Fu : 0u,
                 m4 = up ? 0x0F0F0000u : 0u;
  float acc[NV];
#pragma unroll
  for (int v = 0; v < NV; ++v) acc[v] = 0.0f;

  int slot = 0;
  const int nlast = max(nu, NB) - 1;
  for (int u = 0; u < nu; ++u) {
    // copies issued after tile u: the prologue's NB-1-u, then one per earlier refill
    const int ahead = min(NB - 1, nlast - u);
    if (ahead >= 3) wait_vm<9>();
    else if (ahead == 2) wait_vm<6>();
    else if (ahead == 1) wait_vm<3>();
    else wait_vm<0>();
    const int s = order(u);
    const uint32_t st = stage_base + (uint32_t)slot * kTileBytes;
    u32x4 hd = lds_read16(st + b_hd), q0 = lds_read16(st + b_q), q1 = lds_read16<16>(st + b_q);
    lds_wait(hd, q0, q1);
    // the stage is in registers: refill it with the tile NB super-blocks on
    if (u + NB < nu) mx_issue(rsrc, off, order(u + NB), stage + slot * kTileBytes);
    slot = slot + 1 == NB ? 0 : slot + 1;
    v4i bm[4];
#pragma unroll
    for (int m = 0; m < 2; ++m) {
      const uint32_t qa = m == 0 ? q0.x : q1.x, qb = m == 0 ? q0.y : q1.y, qc = m == 0 ? q0.z : q1.z,
                     qd = m == 0 ? q0.w : q1.w;
      bm[2 * m] = (v4i){(int)(qa & 0x0F0F0F0Fu), (int)(qb & 0x0F0F0F0Fu), (int)hi_codes(qa), (int)hi_codes(qb)};
      bm[2 * m + 1] = (v4i){(int)(qc & 0x0F0F0F0Fu), (int)(qd & 0x0F0F0F0Fu), (int)hi_codes(qc), (int)hi_codes(qd)};
    }
    // scale / min of sub-blocks 2g, 2g+1 and d, dmin (this lane folds group g of tile row j)
    const uint32_t p1 = __builtin_amdgcn_perm(hd.z, hd.y, sel1), p2 = __builtin_amdgcn_perm(hd.w, hd.w, sel2);
    const uint32_t sm = (p1 & m1) | ((p1 >> 2) & m2) | (p2 & m3) | ((p2 >> 4) & m4);
    const float sca = (float)(sm & 0xFFu), scb16 = (float)((sm >> 8) & 0xFFu) * 0.0625f;
    const float mna = (float)((sm >> 16) & 0xFFu), mnb = (float)(sm >> 24);
    const float d = f16lo(hd.x), dmin = f16hi(hd.x);
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      const uint32_t vs = (uint32_t)(v * nsb + s);
      const uint32_t aa = frag_base + vs * kFragBytes + a_rel;
      u32x4 r0 = lds_read16<0>(aa), r1 = lds_read16<16>(aa), mt = lds_read16(meta_base + vs * 64u);
      lds_wait(r0, r1, mt);
      const u32x4 a0 = {r0.x & mlo, r0.y & mlo, r0.x & mhi, r0.y & mhi};
      const u32x4 a1 = {r0.z & mlo, r0.w & mlo, r0.z & mhi, r0.w & mhi};
      const u32x4 a2 = {r1.x & mlo, r1.y & mlo, r1.x & mhi, r1.y & mhi};
      const u32x4 a3 = {r1.z & mlo, r1.w & mlo, r1.z & mhi, r1.w & mhi};
      v4i c = {0, 0, 0, 0};
      c = __builtin_amdgcn_mfma_i32_16x16x64_i8(__builtin_bit_cast(v4i, a0), bm[0], c, 0, 0, 0);
      c = __builtin_amdgcn_mfma_i32_16x16x64_i8(__builtin_bit_cast(v4i, a1), bm[1], c, 0, 0, 0);
      c = __builtin_amdgcn_mfma_i32_16x16x64_i8(__builtin_bit_cast(v4i, a2), bm[2], c, 0, 0, 0);
      c = __builtin_amdgcn_mfma_i32_16x16x64_i8(__builtin_bit_cast(v4i, a3), bm[3], c, 0, 0, 0);
      const int ta = (int)((uint32_t)c[0] << 7) + c[1];                         // sum n q, sub-block 2g
      // meta = [sx, Qa, Qb, 128 Qb]: element values go through __uint_as_float (a bit_cast of a vector
      // element lvalue is miscompiled here: it reads element 0)
      const int tb = (int)((uint32_t)c[2] << 7) + c[3] + (int)mt.w;             // 16 * sum n q, sub-block 2g+1
      const float t = __builtin_fmaf((float)tb, scb16, (float)ta * sca);
      const float w = __builtin_fmaf(__uint_as_float(mt.z), mnb, __uint_as_float(mt.y) * mna);
      acc[v] = __builtin_fmaf(__builtin_fmaf(d, t, -dmin * w), __uint_as_float(mt.x), acc[v]);
    }
  }

  wait_vm<0>();  // repeated prologue tiles may still be in flight: none may land after the wave ends

  // 5. sum over the four groups (lanes j, j+16, j+32, j+48), then over the KQ waves of the tile
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    float sv = acc[v];
    const auto a32 = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(int, sv), __builtin_bit_cast(int, sv), false, false);
    sv = __builtin_bit_cast(float, (int)a32[0]) + __builtin_bit_cast(float, (int)a32[1]);
    const auto a16 = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(int, sv), __builtin_bit_cast(int, sv), false, false);
    acc[v] = __builtin_bit_cast(float, (int)a16[0]) + __builtin_bit_cast(float, (int)a16[1]);
  }
  if (lane < 16) {
#pragma unroll
    for (int v = 0; v < NV; ++v) red[((tq * KQ + kq) * NV + v) * 16 + lane] = acc[v];
  }
  __syncthreads();
  mx_store<EPI>(red, Y, NV, rows, rb, cnt, TQ, KQ, tid);
}

template <int NV, int NB, int TPT, int EPI>
__global__ __launch_bounds__(1024) void k_gemv_mx(const uint8_t* __restrict__ W, const float* __restrict__ X,
                                                  float* __restrict__ Y, int rows, int cols, MxGeo geo,
                                                  const float* __restrict__ NW, float eps) {
  gemv_mx_body<NV, NB, TPT, EPI>(W, X, Y, rows, cols, geo, NW, eps, blockIdx.x);
}

// ---- batched form: 2..8 vectors a launch ------------------------------------------------------
// One v_mfma_i32_16x16x32_i8 per 32-element sub-block of the tile serves 8 vectors:
//  * B (16 columns = weight rows j, K = 32): lane (j, kg) supplies the codes of elements
//    8kg..8kg+7 of sub-block sb: low nibbles (even sb) or high nibbles (odd sb) of qs bytes
//    32(sb/2) + 8kg..8kg+7 of row j, as bytes 0..15 (no offset).
//  * A (16 rows = (vector u, part p), row 2u + p): lane (2u + p, kg) holds qh (p = 0) or ql
//    (p = 1) of vector u at the same elements.  The fragments of one sub-block are 512 bytes,
//    [kg][row] x 8 bytes, so a wave reads them with one conflict-free ds_read_b64.
//  * D: lane (j, r) holds rows 4r..4r+3 = (vector 2r: qh, ql), (vector 2r+1: qh, ql) of column j:
//    the integers sum n*q of sub-block sb for two vectors.
// The lane keeps one accumulator per (vector, group), folds each group exactly as the one-vector
// kernel does (the same integers ta = sum n q of sub-block 2c and tb = 16 sum n q of sub-block
// 2c+1, the same float expression, the same order over super-blocks), combines the groups as
// (g0 + g2) + (g1 + g3) -- the order of that kernel's permlane sums -- and the K-split waves in
// wave order with the same geometry.  So every output is bit-identical to the one-vector kernel's,
// which keeps qvx_qmatmul_n bit-identical to qvx_qmatmul per vector.

constexpr int kSubBytes = 512;  // A fragments of one sub-block for 8 vectors

// LDS: dynamic [fragments: nsb*8*512][meta: nsb*4 groups*8 vectors*16] and a static tile ring
// [16 waves][2][2304].
__host__ __device__ inline size_t mxb_frag_bytes(int nsb) { return (size_t)nsb * 8 * kSubBytes; }
__host__ __device__ inline size_t mxb_meta_bytes(int nsb) { return (size_t)nsb * 4 * 8 * 16; }
__host__ __device__ inline size_t mxb_dyn_bytes(int nsb) { return mxb_frag_bytes(nsb) + mxb_meta_bytes(nsb); }
__host__ __device__ inline size_t mxb_lds_bytes(int nsb) { return mxb_dyn_bytes(nsb) + (size_t)16 * 2 * kTileBytes; }

__device__ inline void mxb_convert(const float4 x0, const float4 x1, int v, int sg, int part, bool store,
                                   uint8_t* frag, float* meta) {
  const XQ8 q = mx_quantize(x0, x1);
  if (store) {
    const int g = sg & 3, s = sg >> 2, sb = 2 * g + (part >> 2), kg = part & 3;
    const uint32_t f = lds_addr(frag) + (uint32_t)((s * 8 + sb) * kSubBytes + (kg * 16 + 2 * v) * 8);
    lds_write8(f, q.h0, q.h1);      // row 2v: qh
    lds_write8(f + 8, q.l0, q.l1);  // row 2v + 1: ql
    const uint32_t mt = lds_addr(meta) + (uint32_t)(((s * 4 + g) * 8 + v) * 16);  // [sx, Qa, Qb, 128 Qb as int]
    if (part == 0) lds_write8(mt, __builtin_bit_cast(uint32_t, q.sx), __builtin_bit_cast(uint32_t, (float)q.sq));
    if (part == 4) lds_write8(mt + 8, __builtin_bit_cast(uint32_t, (float)q.sq), (uint32_t)(128 * q.sq));
  }
}

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
__device__ inline u32x2 lds_read8(uint32_t addr) {
  u32x2 r;
  asm volatile("ds_read_b64 %0, %1" : "=v"(r) : "v"(addr) : "memory");
  return r;
}
__device__ inline void lds_wait5(u32x4& a, u32x2& b, u32x2& c, u32x2& d, u32x2& e) {
  asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(a), "+v"(b), "+v"(c), "+v"(d), "+v"(e)::"memory");
}
__device__ inline void lds_wait16(u32x2 (&a)[8], u32x4 (&m)[8]) {
  asm volatile("s_waitcnt lgkmcnt(0)"
               : "+v"(a[0]), "+v"(a[1]), "+v"(a[2]), "+v"(a[3]), "+v"(a[4]), "+v"(a[5]), "+v"(a[6]), "+v"(a[7]),
                 "+v"(m[0]), "+v"(m[1]), "+v"(m[2]), "+v"(m[3]), "+v"(m[4]), "+v"(m[5]), "+v"(m[6]), "+v"(m[7])::"memory");
}

// Scale / min of sub-blocks 2c, 2c+1 of a Q4_K header (the 6-bit fields, as the one-vector kernel
// unpacks them for its lane group c).
__device__ inline void q4k_group_scales(const u32x4& hd, int c, float& sca, float& scb16, float& mna, float& mnb) {
  const uint32_t jj = 2u * (uint32_t)(c & 1);
  const uint32_t sel1 = jj | (jj + 1) << 8 | (jj + 4) << 16 | (jj + 5) << 24;
  const uint32_t sel2 = jj | (jj + 1) << 8 | jj << 16 | (jj + 1) << 24;
  const bool up = c >= 2;
  const uint32_t m1 = up ? 0u : 0x3F3F3F3Fu, m2 = up ? 0x30303030u : 0u, m3 = up ? 0x00000F0Fu : 0u,
                 m4 = up ? 0x0F0F0000u : 0u;
  const uint32_t p1 = __builtin_amdgcn_perm(hd.z, hd.y, sel1), p2 = __builtin_amdgcn_perm(hd.w, hd.w, sel2);
  const uint32_t sm = (p1 & m1) | ((p1 >> 2) & m2) | (p2 & m3) | ((p2 >> 4) & m4);
  sca = (float)(sm & 0xFFu);
  scb16 = (float)((sm >> 8) & 0xFFu) * 0.0625f;
  mna = (float)((sm >> 16) & 0xFFu);
  mnb = (float)(sm >> 24);
}

// One tile's MFMAs and fold: header hd and codes qq (this lane's row j = lane%16, K block
// r4 = lane/16), A fragments af[sb] of the super-block's eight sub-blocks, activation records
// mf[2c + e] of group c for vectors 2 r4 + e.  acc[e][c] += the group's term, for both vectors.
// Group c of the tile: A fragments a0 / a1 of sub-blocks 2c / 2c+1, records m0 / m1 of vectors
// 2 r4 / 2 r4 + 1 ([sx, Qa, Qb, ...]).
template <typename MT>
__device__ inline void mxb_fold_group(int c, const u32x4& hd, const u32x2& q, const u32x2& a0, const u32x2& a1,
                                      const MT& m0, const MT& m1, float (&acc)[2][4]) {
  const float d = f16lo(hd.x), dmin = f16hi(hd.x);
  const u32x2 bl = {q.x & 0x0F0F0F0Fu, q.y & 0x0F0F0F0Fu};
  const u32x2 bh = {(q.x >> 4) & 0x0F0F0F0Fu, (q.y >> 4) & 0x0F0F0F0Fu};
  const v4i zero = {0, 0, 0, 0};
  const v4i da =
      __builtin_amdgcn_mfma_i32_16x16x32_i8(__builtin_bit_cast(long, a0), __builtin_bit_cast(long, bl), zero, 0, 0, 0);
  const v4i db =
      __builtin_amdgcn_mfma_i32_16x16x32_i8(__builtin_bit_cast(long, a1), __builtin_bit_cast(long, bh), zero, 0, 0, 0);
  float sca, scb16, mna, mnb;
  q4k_group_scales(hd, c, sca, scb16, mna, mnb);
#pragma unroll
  for (int e = 0; e < 2; ++e) {
    const MT mt = e == 0 ? m0 : m1;
    const int ta = (int)((uint32_t)da[2 * e] << 7) + da[2 * e + 1];                      // sum n q, sub-block 2c
    const int tb = (int)((((uint32_t)db[2 * e] << 7) + (uint32_t)db[2 * e + 1]) << 4);  // 16 sum n q, 2c+1
    const float t = __builtin_fmaf((float)tb, scb16, (float)ta * sca);
    const float w = __builtin_fmaf(__uint_as_float(mt.z), mnb, __uint_as_float(mt.y) * mna);
    acc[e][c] = __builtin_fmaf(__builtin_fmaf(d, t, -dmin * w), __uint_as_float(mt.x), acc[e][c]);
  }
}

template <typename MT>
__device__ inline void mxb_fold(const u32x4& hd, const u32x2 (&qq)[4], const u32x2 (&af)[8], const MT (&mf)[8],
                                float (&acc)[2][4]) {
#pragma unroll
  for (int c = 0; c < 4; ++c) mxb_fold_group(c, hd, qq[c], af[2 * c], af[2 * c + 1], mf[2 * c], mf[2 * c + 1], acc);
}

// EPI as for k_gemv_mx.
template <int TPT, int EPI>
__global__ __launch_bounds__(1024) void k_gemv_mxb(const uint8_t* __restrict__ W, const float* __restrict__ X,
                                                   float* __restrict__ Y, int rows, int cols, int nv, MxGeo geo,
                                                   const float* __restrict__ NW, float eps) {
  constexpr int NB = 2;
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  __shared__ __attribute__((aligned(16))) uint8_t ring[16 * NB * kTileBytes];
  __shared__ __attribute__((aligned(16))) float sqp[(EPI & EPI_NORM) ? 8 * kNormMaxChunks : 4];  // chunk sums
  const int nsb = geo.nsb, TQ = geo.TQ, KQ = geo.KQ;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  uint8_t* frag = lds;
  float* meta = reinterpret_cast<float*>(lds + mxb_frag_bytes(nsb));
  QVX_LDS uint8_t* stage = (QVX_LDS uint8_t*)(ring + wave * NB * kTileBytes);

  const int b = blockIdx.x;
  const int rb = b * geo.base + geo.unit * min(b, geo.rem), cnt = geo.base + (b < geo.rem ? geo.unit : 0);
  const int tq = wave % TQ, kq = wave / TQ;
  const int s0 = kq * nsb / KQ, s1 = (kq + 1) * nsb / KQ, nu = s1 - s0;
  const SbOrder order(kq, KQ, s0, s1);

  // 1. activations -> A fragments (waves with conversion tasks), before any copy.  Every round's
  // loads are issued before the first conversion: the fragment stores (inline asm with a memory
  // clobber) would otherwise keep each round's loads behind the previous round's stores, one memory
  // latency per round.
  const int per = nsb * 32, ntask = nv * per;
  float4 xa[TPT], xb[TPT], wa[TPT], wb[TPT];
#pragma unroll
  for (int k = 0; k < TPT; ++k) {
    if (1024 * k + 64 * wave < ntask) {
      const int t = min(tid + 1024 * k, ntask - 1), v = t / per, r = t - v * per;
      const float4* src = reinterpret_cast<const float4*>(X + (size_t)v * cols + 8 * r);
      xa[k] = src[0];
      xb[k] = src[1];
      if constexpr ((EPI & EPI_NORM) != 0) {
        wa[k] = reinterpret_cast<const float4*>(NW + 8 * r)[0];
        wb[k] = reinterpret_cast<const float4*>(NW + 8 * r)[1];
      }
    }
  }
  if constexpr ((EPI & EPI_NORM) != 0) mx_norm<TPT>(xa, xb, wa, wb, tid, per, ntask, cols, eps, sqp);
#pragma unroll
  for (int k = 0; k < TPT; ++k) {
    if (1024 * k + 64 * wave < ntask) {
      const int t0 = tid + 1024 * k, t = min(t0, ntask - 1), v = t / per, r = t - v * per;
      mxb_convert(xa[k], xb[k], v, r >> 3, r & 7, t0 < ntask, frag, meta);
    }
  }

  // 2. prologue copies (as the one-vector kernel)
  const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(W + (size_t)rb * geo.row_bytes), (short)0, (int)((uint32_t)cnt * geo.row_bytes), (int)kRsrcWord3);
  uint32_t off[3];
#pragma unroll
  for (int k = 0; k < 3; ++k) {
    const uint32_t p = k < 2 ? (uint32_t)(1024 * k + 16 * lane) : (uint32_t)(2048 + 4 * lane);
    const uint32_t r = p / (uint32_t)kSB, c = p - (uint32_t)kSB * r;
    off[k] = __umul24(16u * (uint32_t)tq + r, geo.row_bytes) + c;
  }
#pragma unroll
  for (int u = 0; u < NB; ++u) mx_issue(rsrc, off, nu > 0 ? order(min(u, nu - 1)) : s0, stage + u * kTileBytes);

  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's fragment stores
  __builtin_amdgcn_s_barrier();

  // 3. tiles
  const int j = lane & 15, r4 = lane >> 4;  // B column (tile row) and K block; D rows 4 r4..4 r4+3
  const uint32_t b_hd = kSB * j, b_q = kSB * j + 16 + 8 * r4;
  const uint32_t frag_base = lds_addr(frag) + 8u * (uint32_t)lane;
  const uint32_t meta_base = lds_addr(meta) + 32u * (uint32_t)r4;  // vectors 2 r4, 2 r4 + 1
  const uint32_t stage_base = (uint32_t)(uintptr_t)stage;
  float acc[2][4];
#pragma unroll
  for (int e = 0; e < 2; ++e)
#pragma unroll
    for (int c = 0; c < 4; ++c) acc[e][c] = 0.0f;

  int slot = 0;
  const int nlast = max(nu, NB) - 1;
  for (int u = 0; u < nu; ++u) {
    if (min(NB - 1, nlast - u) >= 1) wait_vm<3>();
    else wait_vm<0>();
    const int s = order(u);
    const uint32_t st = stage_base + (uint32_t)slot * kTileBytes;
    u32x4 hd = lds_read16(st + b_hd);
    u32x2 q0 = lds_read8(st + b_q), q1 = lds_read8(st + b_q + 32), q2 = lds_read8(st + b_q + 64),
          q3 = lds_read8(st + b_q + 96);
    lds_wait5(hd, q0, q1, q2, q3);
    if (u + NB < nu) mx_issue(rsrc, off, order(u + NB), stage + slot * kTileBytes);
    slot = slot + 1 == NB ? 0 : slot + 1;
    const u32x2 qq[4] = {q0, q1, q2, q3};
    // every A fragment and activation record of the tile in one round trip
    u32x2 af[8];
    u32x4 mf[8];
    const uint32_t fa = frag_base + (uint32_t)(s * 8) * kSubBytes;
    const uint32_t ma = meta_base + (uint32_t)(s * 4 * 8) * 16u;
#pragma unroll
    for (int k = 0; k < 8; ++k) af[k] = lds_read8(fa + (uint32_t)k * kSubBytes);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      mf[2 * c] = lds_read16(ma + (uint32_t)c * 128u);
      mf[2 * c + 1] = lds_read16<16>(ma + (uint32_t)c * 128u);
    }
    lds_wait16(af, mf);
    mxb_fold(hd, qq, af, mf, acc);
  }

  wait_vm<0>();

  // 4. groups as (g0 + g2) + (g1 + g3), then the KQ waves of the tile in wave order
  __syncthreads();
  float* red = reinterpret_cast<float*>(ring);  // [tq][kq][v][16]
#pragma unroll
  for (int e = 0; e < 2; ++e) {
    const int v = 2 * r4 + e;
    if (v < nv) red[((tq * KQ + kq) * nv + v) * 16 + j] = (acc[e][0] + acc[e][2]) + (acc[e][1] + acc[e][3]);
  }
  __syncthreads();
  mx_store<EPI>(red, Y, nv, rows, rb, cnt, TQ, KQ, tid);
}

// ---- batched form for long rows -----------------------------------------------------------------
// Where the batched form's fragments for a whole row do not fit in LDS, each wave converts the
// activations of one super-block just before it folds that super-block, into a private buffer with
// the batched form's layout ([sb][kg][row] fragments, [g][v] records: 4.5 KB), so LDS use does not
// depend on K.  The next super-block's activations are loaded into registers while the current
// one is folded: issue order x(s0) c(s0) c(s0+1) | x(s0+1) c(s0+2) | ..., so at step u the wave
// needs x(u) and c(u) and only c(u+1) may still be in flight (vmcnt 3); the last two steps are
// peeled so that every wait is exact.  The geometry, the conversion (the same 8-lane task groups)
// and the fold are the batched form's, so outputs stay bit-identical to the one-vector kernel's.
// Waves whose tiles share super-blocks (TQ > 1) convert them again each: the form is meant for
// the long-row shapes, where rows <= 16 * 256 and TQ = 1.

constexpr int kJitBytes = 8 * kSubBytes + 4 * 8 * 16;  // one super-block: fragments + records

// NVT conversion rounds per lane: task t = lane + 64 k = 8 elements (vector t/32, group (t%32)/8,
// part t%8); the vector index is clamped for the loads, the stores skip vectors >= nv.
template <int NVT>
struct XRegs {
  float4 a[NVT], b[NVT];
};

template <int NVT>
__device__ inline void mxj_load(const float* __restrict__ X, int cols, int nv, int s, int lane, XRegs<NVT>& x) {
#pragma unroll
  for (int k = 0; k < NVT; ++k) {
    const int t = lane + 64 * k, v = min(t >> 5, nv - 1), r = t & 31;
    const float4* p = reinterpret_cast<const float4*>(X + (size_t)v * cols + 256 * s + 8 * r);
    x.a[k] = p[0];
    x.b[k] = p[1];
  }
}

template <int NVT>
__device__ inline void mxj_convert(const XRegs<NVT>& x, int nv, int lane, uint8_t* frag, float* meta) {
#pragma unroll
  for (int k = 0; k < NVT; ++k) {
    const int t = lane + 64 * k, v = t >> 5, r = t & 31;
    mxb_convert(x.a[k], x.b[k], v, r >> 3, r & 7, v < nv, frag, meta);
  }
}

typedef uint32_t u32x3 __attribute__((ext_vector_type(3)));
template <int OFF = 0>
__device__ inline u32x3 lds_read12(uint32_t addr) {
  u32x3 r;
  asm volatile("ds_read_b96 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "i"(OFF) : "memory");
  return r;
}

__device__ inline void lds_wait13(u32x4& h, u32x2 (&q)[4], u32x2 (&a)[4], u32x3 (&m)[4]) {
  asm volatile("s_waitcnt lgkmcnt(0)"
               : "+v"(h), "+v"(q[0]), "+v"(q[1]), "+v"(q[2]), "+v"(q[3]), "+v"(a[0]), "+v"(a[1]), "+v"(a[2]),
                 "+v"(a[3]), "+v"(m[0]), "+v"(m[1]), "+v"(m[2]), "+v"(m[3])::"memory");
}
__device__ inline void lds_wait8(u32x2 (&a)[4], u32x3 (&m)[4]) {
  asm volatile("s_waitcnt lgkmcnt(0)"
               : "+v"(a[0]), "+v"(a[1]), "+v"(a[2]), "+v"(a[3]), "+v"(m[0]), "+v"(m[1]), "+v"(m[2]), "+v"(m[3])::"memory");
}

// A fragments of sub-blocks 4h..4h+3 and the records of groups 2h, 2h+1 (this lane's two vectors).
__device__ inline void mxj_read_half(int h, uint32_t fa, uint32_t ma, u32x2 (&a)[4], u32x3 (&m)[4]) {
#pragma unroll
  for (int k = 0; k < 4; ++k) a[k] = lds_read8(fa + (uint32_t)(4 * h + k) * kSubBytes);
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    m[2 * c] = lds_read12(ma + (uint32_t)(2 * h + c) * 128u);
    m[2 * c + 1] = lds_read12<16>(ma + (uint32_t)(2 * h + c) * 128u);
  }
}

template <int NVT>
__global__ __launch_bounds__(1024) void k_gemv_mxj(const uint8_t* __restrict__ W, const float* __restrict__ X,
                                                   float* __restrict__ Y, int rows, int cols, int nv, MxGeo geo) {
  constexpr int NB = 2;
  __shared__ __attribute__((aligned(16))) uint8_t ring[16 * NB * kTileBytes];
  __shared__ __attribute__((aligned(16))) uint8_t jit[16 * kJitBytes];
  const int nsb = geo.nsb, TQ = geo.TQ, KQ = geo.KQ;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  uint8_t* frag = jit + wave * kJitBytes;
  float* meta = reinterpret_cast<float*>(frag + 8 * kSubBytes);
  QVX_LDS uint8_t* stage = (QVX_LDS uint8_t*)(ring + wave * NB * kTileBytes);

  const int b = blockIdx.x;
  const int rb = b * geo.base + geo.unit * min(b, geo.rem), cnt = geo.base + (b < geo.rem ? geo.unit : 0);
  const int tq = wave % TQ, kq = wave / TQ;
  const int s0 = kq * nsb / KQ, s1 = (kq + 1) * nsb / KQ, nu = s1 - s0;
  const SbOrder order(kq, KQ, s0, s1);

  const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(W + (size_t)rb * geo.row_bytes), (short)0, (int)((uint32_t)cnt * geo.row_bytes), (int)kRsrcWord3);
  uint32_t off[3];
#pragma unroll
  for (int k = 0; k < 3; ++k) {
    const uint32_t p = k < 2 ? (uint32_t)(1024 * k + 16 * lane) : (uint32_t)(2048 + 4 * lane);
    const uint32_t r = p / (uint32_t)kSB, c = p - (uint32_t)kSB * r;
    off[k] = __umul24(16u * (uint32_t)tq + r, geo.row_bytes) + c;
  }

  const int j = lane & 15, r4 = lane >> 4;  // B column (tile row) and K block; D rows 4 r4..4 r4+3
  const uint32_t b_hd = kSB * j, b_q = kSB * j + 16 + 8 * r4;
  const uint32_t fa = lds_addr(frag) + 8u * (uint32_t)lane;
  const uint32_t ma = lds_addr(meta) + 32u * (uint32_t)r4;  // vectors 2 r4, 2 r4 + 1
  const uint32_t stage_base = (uint32_t)(uintptr_t)stage;
  float acc[2][4];
#pragma unroll
  for (int e = 0; e < 2; ++e)
#pragma unroll
    for (int c = 0; c < 4; ++c) acc[e][c] = 0.0f;
  XRegs<NVT> x;

  // step u: super-block order(u) is in stage u & 1 and its activations in x
#define QVX_MXJ_STEP(U, WAITN, NEXT_X, NEXT_COPY)                                                    \
  {                                                                                                  \
    wait_vm<WAITN>();                                                                                \
    mxj_convert<NVT>(x, nv, lane, frag, meta);                                                       \
    const uint32_t st = stage_base + (uint32_t)((U) & 1) * kTileBytes;                              \
    u32x4 hd = lds_read16(st + b_hd);                                                                \
    u32x2 qq[4];                                                                                     \
    _Pragma("unroll") for (int c = 0; c < 4; ++c) qq[c] = lds_read8(st + b_q + 32u * (uint32_t)c);  \
    u32x2 a0[4], a1[4];                                                                              \
    u32x3 m0[4], m1[4];                                                                              \
    mxj_read_half(0, fa, ma, a0, m0);                                                                \
    lds_wait13(hd, qq, a0, m0);                                                                      \
    if (NEXT_X) mxj_load<NVT>(X, cols, nv, order((U) + 1), lane, x);                                 \
    if (NEXT_COPY) mx_issue(rsrc, off, order((U) + 2), stage + ((U) & 1) * kTileBytes);              \
    mxj_read_half(1, fa, ma, a1, m1);                                                                \
    mxb_fold_group(0, hd, qq[0], a0[0], a0[1], m0[0], m0[1], acc);                                   \
    mxb_fold_group(1, hd, qq[1], a0[2], a0[3], m0[2], m0[3], acc);                                   \
    lds_wait8(a1, m1);                                                                               \
    mxb_fold_group(2, hd, qq[2], a1[0], a1[1], m1[0], m1[1], acc);                                   \
    mxb_fold_group(3, hd, qq[3], a1[2], a1[3], m1[2], m1[3], acc);                                   \
  }

  if (nu >= 2) {
    mxj_load<NVT>(X, cols, nv, order(0), lane, x);
    mx_issue(rsrc, off, order(0), stage);
    mx_issue(rsrc, off, order(1), stage + kTileBytes);
    int u = 0;
    for (; u + 2 < nu; ++u) QVX_MXJ_STEP(u, 3, true, true)
    QVX_MXJ_STEP(u, 3, true, false)
    ++u;
    QVX_MXJ_STEP(u, 0, false, false)
  } else if (nu == 1) {
    mxj_load<NVT>(X, cols, nv, s0, lane, x);
    mx_issue(rsrc, off, s0, stage);
    QVX_MXJ_STEP(0, 0, false, false)
  }
#undef QVX_MXJ_STEP
  wait_vm<0>();

  // groups as (g0 + g2) + (g1 + g3), then the KQ waves of the tile in wave order
  __syncthreads();
  float* red = reinterpret_cast<float*>(ring);  // [tq][kq][v][16]
#pragma unroll
  for (int e = 0; e < 2; ++e) {
    const int v = 2 * r4 + e;
    if (v < nv) red[((tq * KQ + kq) * nv + v) * 16 + j] = (acc[e][0] + acc[e][2]) + (acc[e][1] + acc[e][3]);
  }
  __syncthreads();
  for (int o = tid; o < TQ * nv * 16; o += 1024) {
    const int t = o / (nv * 16), v = (o >> 4) % nv, r = o & 15;
    const int row = 16 * t + r;
    if (row < cnt) {
      float sum = 0.0f;
      for (int k = 0; k < KQ; ++k) sum += red[((t * KQ + k) * nv + v) * 16 + r];
      Y[(size_t)v * rows + rb + row] = sum;
    }
  }
}

constexpr int kCUs = 256;
constexpr size_t kLdsMax = kLdsPerCU;

template <int NV, int NB, int TPT, int EPI>
static bool launch_mx(const void* w, const float* X, float* Y, int rows, int cols, const MxGeo& geo, int nwg,
                      const GemvEpi& epi, hipStream_t s) {
  auto kern = &k_gemv_mx<NV, NB, TPT, EPI>;
  const size_t lds = mx_dyn_bytes(NV, geo.nsb);
  static LdsLimit lim;
  if (!lds_ready(reinterpret_cast<const void*>(kern), lim, lds)) return false;
  kern<<<(unsigned)nwg, 1024u, lds, s>>>(static_cast<const uint8_t*>(w), X, Y, rows, cols, geo, epi.norm_w, epi.eps);
  return true;
}

template <int NV, int NB, int TPT>
static bool launch_mx_epi(const void* w, const float* X, float* Y, int rows, int cols, const MxGeo& geo, int nwg,
                          const GemvEpi& epi, hipStream_t s) {
  switch (epi.flags()) {
    case 0: return launch_mx<NV, NB, TPT, 0>(w, X, Y, rows, cols, geo, nwg, epi, s);
    case EPI_NORM: return launch_mx<NV, NB, TPT, EPI_NORM>(w, X, Y, rows, cols, geo, nwg, epi, s);
    case EPI_SWIGLU: return launch_mx<NV, NB, TPT, EPI_SWIGLU>(w, X, Y, rows, cols, geo, nwg, epi, s);
    default: return launch_mx<NV, NB, TPT, EPI_NORM | EPI_SWIGLU>(w, X, Y, rows, cols, geo, nwg, epi, s);
  }
}

// Two stages per wave (two tiles in flight behind the one being folded).  Deeper rings only
// lengthen each wave's copy issue before the fragment barrier, as issue stalls once the CU's
// request queue is full.  TPT = activation conversion tasks per thread.
template <int NV>
static bool launch_mx_nv(const void* w, const float* X, float* Y, int rows, int cols, const MxGeo& geo, int nwg,
                         const GemvEpi& epi, hipStream_t s) {
  const int tpt = (NV * geo.nsb * 32 + 1023) / 1024;
  if (tpt <= 1) return launch_mx_epi<NV, 2, 1>(w, X, Y, rows, cols, geo, nwg, epi, s);
  if (tpt <= 2) return launch_mx_epi<NV, 2, 2>(w, X, Y, rows, cols, geo, nwg, epi, s);
  return launch_mx_epi<NV, 2, 4>(w, X, Y, rows, cols, geo, nwg, epi, s);
}

// Launch geometry shared by all three forms (the batched forms' bit-identity rests on it): one
// workgroup of 16 waves per CU; tiles of 16 rows; TQ tiles x KQ K-splits per workgroup.  Rows are
// dealt in whole units (unit = 32 for a fused SwiGLU launch, rows % 32 == 0, so every workgroup
// holds whole (gate, up) tile pairs).
static int mx_geometry(int rows, int cols, size_t row_bytes, MxGeo& geo, int unit = 1) {
  geo.nsb = cols / 256;
  geo.row_bytes = (uint32_t)row_bytes;
  geo.unit = unit;
  const int units = rows / unit;
  int64_t nwg = std::min<int64_t>(kCUs, ((int64_t)rows + 15) / 16);
  nwg = std::max<int64_t>(nwg, ((int64_t)rows + 255) / 256);
  nwg = std::min<int64_t>(nwg, units);
  geo.base = (int)(units / nwg) * unit;
  geo.rem = (int)(units % nwg);
  const int per = geo.base + (geo.rem ? unit : 0);
  int tq = 1;
  while (16 * tq < per) tq <<= 1;
  geo.TQ = tq;
  geo.KQ = 16 / tq;
  return (int)nwg;
}

template <int TPT, int EPI>
static bool launch_mxb(const void* w, const float* X, float* Y, int nv, int rows, int cols, const MxGeo& geo, int nwg,
                       const GemvEpi& epi, hipStream_t s) {
  auto kern = &k_gemv_mxb<TPT, EPI>;
  const size_t lds = mxb_dyn_bytes(geo.nsb);
  static LdsLimit lim;
  if (!lds_ready(reinterpret_cast<const void*>(kern), lim, lds)) return false;
  kern<<<(unsigned)nwg, 1024u, lds, s>>>(static_cast<const uint8_t*>(w), X, Y, rows, cols, nv, geo, epi.norm_w,
                                         epi.eps);
  return true;
}

template <int TPT>
static bool launch_mxb_epi(const void* w, const float* X, float* Y, int nv, int rows, int cols, const MxGeo& geo,
                           int nwg, const GemvEpi& epi, hipStream_t s) {
  switch (epi.flags()) {
    case 0: return launch_mxb<TPT, 0>(w, X, Y, nv, rows, cols, geo, nwg, epi, s);
    case EPI_NORM: return launch_mxb<TPT, EPI_NORM>(w, X, Y, nv, rows, cols, geo, nwg, epi, s);
    case EPI_SWIGLU: return launch_mxb<TPT, EPI_SWIGLU>(w, X, Y, nv, rows, cols, geo, nwg, epi, s);
    default: return launch_mxb<TPT, EPI_NORM | EPI_SWIGLU>(w, X, Y, nv, rows, cols, geo, nwg, epi, s);
  }
}

template <int NVT>
static bool launch_mxj(const uint8_t* w, const float* X, float* Y, int nv, int rows, int cols, const MxGeo& geo,
                       int nwg, hipStream_t s) {
  auto kern = &k_gemv_mxj<NVT>;
  static LdsLimit lim;
  if (!lds_ready(reinterpret_cast<const void*>(kern), lim, 0)) return false;
  kern<<<(unsigned)nwg, 1024u, 0, s>>>(w, X, Y, rows, cols, nv, geo);
  return true;
}


// ---- grouped launch: several one-vector GEMVs of the same activations -------------------------
// Members share x.  Q4_K members run the matrix-core body above, a Q6_K member the VALU body of
// qvx_gemv_valu.hpp, each with the geometry its own launch would take (mx_geometry / valu_grid), so
// every row's arithmetic and summation order are its standalone kernel's and each member's outputs
// are bit-identical to its own qvx_qmatmul.  Workgroups are numbered member after member, the Q6_K
// member's first: they are the longest-latency ones (one row each, every lane's bytes in one load
// round), so they start while the matrix-core workgroups still stream.  One launch pays the
// dispatch ramp and the drain once for the whole group.
constexpr int kGroupMx = 4;  // Q4_K members a launch

struct GroupMx {
  const uint8_t* w;
  float* y;
  int rows, nwg;
  MxGeo geo;
};
struct GroupArgs {
  GroupMx mx[kGroupMx];
  int nmx;
  const uint8_t* vw;  // the Q6_K member (vnwg = 0: none)
  float* vy;
  int vrows, vnwg;
  Geo vgeo;
};

// NORM: every member takes rmsnorm(x, NW, eps) as its activations, folded into each body's
// conversion as in its standalone kernel (qvx_qmatmul_n_rmsnorm's arithmetic).
template <int TPT, int RMAX, bool CH, bool NORM>
__global__ __launch_bounds__(1024) void k_gemv_group(const float* __restrict__ X, int cols, GroupArgs a,
                                                     const float* __restrict__ NW, float eps) {
  int b = blockIdx.x;
  if (b < a.vnwg) {
    constexpr int PF = prefetch_rows<T_Q6_K, 1>() < RMAX ? prefetch_rows<T_Q6_K, 1>() : RMAX;
    const int sp = a.vgeo.Sp, t = threadIdx.x;
    gemv_valu_body<T_Q6_K, 1, RMAX, TPT, PF, CH, NORM>(a.vw, X, a.vy, a.vrows, cols, a.vgeo, NW, eps, b, t % sp,
                                                        t / sp);
    return;
  }
  b -= a.vnwg;
  int i = 0;
  while (i + 1 < a.nmx && b >= a.mx[i].nwg) {
    b -= a.mx[i].nwg;
    ++i;
  }
  gemv_mx_body<1, 2, TPT, NORM ? EPI_NORM : 0>(a.mx[i].w, X, a.mx[i].y, a.mx[i].rows, cols, a.mx[i].geo, NW, eps,
                                               b);
}

template <int TPT, int RMAX, bool CH, bool NORM>
static bool launch_group_t(const float* X, int cols, const GroupArgs& a, int nwg, const GemvEpi& epi,
                           hipStream_t s) {
  auto kern = &k_gemv_group<TPT, RMAX, CH, NORM>;
  const size_t lds = std::max(mx_dyn_bytes(1, cols / 256), a.vnwg ? gemv_lds_bytes<T_Q6_K>(1, a.vgeo.S) : 0);
  static LdsLimit lim;
  if (!lds_ready(reinterpret_cast<const void*>(kern), lim, lds)) return false;
  kern<<<(unsigned)nwg, 1024u, lds, s>>>(X, cols, a, epi.norm_w, epi.eps);
  return true;
}

// Rows per VALU group, rounded up to an instantiated chunk (a chunk longer than the group's rows
// clamps the extra loads to its last row and drops their results, so the outputs do not change).
template <int TPT, bool NORM>
static bool launch_group_tpt(const float* X, int cols, const GroupArgs& a, int nwg, int per_group,
                             const GemvEpi& epi, hipStream_t s) {
  if (per_group <= 1) return launch_group_t<TPT, 1, false, NORM>(X, cols, a, nwg, epi, s);
  if (per_group <= 2) return launch_group_t<TPT, 2, false, NORM>(X, cols, a, nwg, epi, s);
  if (per_group <= 4) return launch_group_t<TPT, 4, false, NORM>(X, cols, a, nwg, epi, s);
  if (per_group <= 8) return launch_group_t<TPT, 8, false, NORM>(X, cols, a, nwg, epi, s);
  return launch_group_t<TPT, 8, true, NORM>(X, cols, a, nwg, epi, s);
}

}  // namespace

// 1 if the fused prologue / epilogue can run on this shape: the norm needs whole 512-element
// chunks (at most kNormMaxChunks), SwiGLU whole 32-row (gate, up) groups.
bool mx_epi_supported(const GemvEpi& epi, int rows, int cols) {
  if (epi.norm_w && (cols % kNormChunk != 0 || cols / kNormChunk > kNormMaxChunks)) return false;
  if (epi.swiglu && rows % 32 != 0) return false;
  return true;
}

// 1 if the batched form takes `cols` (its 8-vector fragments fit in LDS with the tile ring).
int gemv_mxb_supported(int cols) {
  if (cols <= 0 || cols % 256 != 0) return 0;
  const int nsb = cols / 256;
  return mxb_lds_bytes(nsb) <= kLdsMax && (8 * nsb * 32 + 1023) / 1024 <= 4 ? 1 : 0;
}

// Q4_K GEMV on the matrix cores, 1 <= nvec <= 8 vectors, batched form.  Returns false, having
// launched nothing, when the shape is not handled here.
bool launch_gemv_mxb_q4k(const void* w, const float* X, float* Y, int nvec, int rows, int cols, size_t row_bytes,
                         const GemvEpi& epi, hipStream_t s) {
  if (!gemv_mxb_supported(cols) || nvec < 1 || nvec > 8 || row_bytes >= (1u << 24)) return false;
  if (!mx_epi_supported(epi, rows, cols)) return false;
  MxGeo geo{};
  const int nwg = mx_geometry(rows, cols, row_bytes, geo, epi.swiglu ? 32 : 1);
  const int tpt = (nvec * geo.nsb * 32 + 1023) / 1024;
  if (tpt <= 1) return launch_mxb_epi<1>(w, X, Y, nvec, rows, cols, geo, nwg, epi, s);
  if (tpt <= 2) return launch_mxb_epi<2>(w, X, Y, nvec, rows, cols, geo, nwg, epi, s);
  return launch_mxb_epi<4>(w, X, Y, nvec, rows, cols, geo, nwg, epi, s);
}

// 1 if the long-row batched form takes `cols`: whole super-blocks, and the one-vector kernel takes
// the same shape (the form's outputs are bit-identical to that kernel's, which single-vector calls
// run).
int gemv_mxj_supported(int cols);

// Q4_K GEMV on the matrix cores, 1 <= nvec <= 8 vectors, long-row batched form (LDS use
// independent of K).  Returns false, having launched nothing, when the shape is not handled here.
bool launch_gemv_mxj_q4k(const void* w, const float* X, float* Y, int nvec, int rows, int cols, size_t row_bytes,
                         hipStream_t s) {
  if (!gemv_mxj_supported(cols) || nvec < 1 || nvec > 8 || row_bytes >= (1u << 24)) return false;
  MxGeo geo{};
  const int nwg = mx_geometry(rows, cols, row_bytes, geo);
  auto* wp = static_cast<const uint8_t*>(w);
  switch ((nvec + 1) / 2) {
    case 1: return launch_mxj<1>(wp, X, Y, nvec, rows, cols, geo, nwg, s);
    case 2: return launch_mxj<2>(wp, X, Y, nvec, rows, cols, geo, nwg, s);
    case 3: return launch_mxj<3>(wp, X, Y, nvec, rows, cols, geo, nwg, s);
    default: return launch_mxj<4>(wp, X, Y, nvec, rows, cols, geo, nwg, s);
  }
}

// Largest vector count one launch takes for a row of `cols` columns (LDS budget), 0 if the shape
// is not handled here.
int gemv_mx_max_nv(int cols) {
  if (cols <= 0 || cols % 256 != 0) return 0;
  const int nsb = cols / 256;
  for (int nv = 8; nv >= 1; --nv)
    if (mx_lds_bytes(nv, nsb, 2) <= kLdsMax && (nv * nsb * 32 + 1023) / 1024 <= 4) return nv;
  return 0;
}

// Q4_K GEMV on the matrix cores for 1 <= nvec <= gemv_mx_max_nv(cols).  Returns false, having
// launched nothing, when the shape is not handled here.
bool launch_gemv_mx_q4k(const void* w, const float* X, float* Y, int nvec, int rows, int cols, size_t row_bytes,
                        const GemvEpi& epi, hipStream_t s) {
  const int maxnv = gemv_mx_max_nv(cols);
  if (maxnv == 0 || nvec < 1 || nvec > maxnv || row_bytes >= (1u << 24)) return false;
  if (!mx_epi_supported(epi, rows, cols)) return false;
  MxGeo geo{};
  const int nwg = mx_geometry(rows, cols, row_bytes, geo, epi.swiglu ? 32 : 1);
  switch (nvec) {
    case 1: return launch_mx_nv<1>(w, X, Y, rows, cols, geo, nwg, epi, s);
    case 2: return launch_mx_nv<2>(w, X, Y, rows, cols, geo, nwg, epi, s);
    case 3: return launch_mx_nv<3>(w, X, Y, rows, cols, geo, nwg, epi, s);
    case 4: return launch_mx_nv<4>(w, X, Y, rows, cols, geo, nwg, epi, s);
    case 5: return launch_mx_nv<5>(w, X, Y, rows, cols, geo, nwg, epi, s);
    case 6: return launch_mx_nv<6>(w, X, Y, rows, cols, geo, nwg, epi, s);
    case 7: return launch_mx_nv<7>(w, X, Y, rows, cols, geo, nwg, epi, s);
    default: return launch_mx_nv<8>(w, X, Y, rows, cols, geo, nwg, epi, s);
  }
}

int gemv_mxj_supported(int cols) {
  return cols > 0 && cols % 256 == 0 && gemv_mx_max_nv(cols) >= 1 ? 1 : 0;
}


// Grouped one-vector GEMV over members that share x (k_gemv_group): up to kGroupMx Q4_K members
// on the matrix-core kernel and at most one Q6_K member on the VALU kernel, all 16-byte aligned
// with 16-byte row pitches (the operands the standalone fast kernels take), optionally on
// rmsnorm(x) (epi.norm_w; no SwiGLU).  Returns false, having launched nothing, when a member or the
// epilogue is outside that set: the caller then runs the members one by one.
bool launch_gemv_group(const GemvMember* m, int n, const float* X, int cols, const GemvEpi& epi, hipStream_t s) {
  if (n < 1 || gemv_mx_max_nv(cols) < 1 || (cols / 256 * 32 + 1023) / 1024 > 2) return false;
  if (epi.swiglu || !mx_epi_supported(epi, 0, cols)) return false;
  GroupArgs a{};
  int nwg = 0, per_group = 0;
  for (int i = 0; i < n; ++i) {
    if (m[i].type == T_Q4_K && a.nmx < kGroupMx && m[i].row_bytes < (1u << 24)) {
      GroupMx& g = a.mx[a.nmx++];
      g.w = static_cast<const uint8_t*>(m[i].w);
      g.y = m[i].y;
      g.rows = m[i].rows;
      g.nwg = mx_geometry(m[i].rows, cols, m[i].row_bytes, g.geo);
      nwg += g.nwg;
    } else if (m[i].type == T_Q6_K && a.vnwg == 0) {
      Geo geo{};
      if (!geometry<T_Q6_K>(cols, m[i].row_bytes, geo) || geo.Sp * geo.G != 1024 ||
          (geo.S * 2 * Lane<T_Q6_K>::kR + 1023) / 1024 != (cols / 256 * 32 + 1023) / 1024)
        return false;  // a full 1024-thread workgroup, and the group's conversion-task count its own
      a.vw = static_cast<const uint8_t*>(m[i].w);
      a.vy = m[i].y;
      a.vrows = m[i].rows;
      a.vnwg = valu_grid(m[i].rows, geo, per_group);
      a.vgeo = geo;
      nwg += a.vnwg;
    } else {
      return false;
    }
  }
  if (a.nmx == 0) return false;
  const bool tpt1 = (cols / 256 * 32 + 1023) / 1024 <= 1;
  if (epi.norm_w)
    return tpt1 ? launch_group_tpt<1, true>(X, cols, a, nwg, per_group, epi, s)
                : launch_group_tpt<2, true>(X, cols, a, nwg, per_group, epi, s);
  return tpt1 ? launch_group_tpt<1, false>(X, cols, a, nwg, per_group, epi, s)
              : launch_group_tpt<2, false>(X, cols, a, nwg, per_group, epi, s);
}


// ---- many vectors: one weight pass per call -----------------------------------------------------
// qvx_qmatmul_n at encoder and prefill batch sizes (nvec in the tens to thousands) streams the
// weights once per 64 vectors instead of once per 8, with every output bit-identical to the
// one-vector kernel's (the reference's promise for qmatmulN, runtime/include/qorvix/runtime/
// qmatmul.hpp:31-32).  Two launches:
//  * k_q4k_many_conv converts every 64-element group of every vector once, with the shared quantiser
//    mx_quantize (the same 8-lane task groups), into a workspace: A fragments [v][s][sb][part][32 B]
//    (qh bytes of sub-block sb's 32 elements, then its ql bytes) and records [v][s][g] = (sx, Qa, Qb).
//  * k_gemv_q4k_many: a wave owns 32 weight rows x 16 vectors and one or more K ranges (the launch
//    shape, many_shape, decides how the tile's vectors and ranges spread over waves and workgroups).
//    Per sub-block one v_mfma_i32_32x32x32_i8 takes A = 32 rows (vector, qh / ql) x 32
//    elements and B = the 32 rows' codes (low nibbles of the group's qs bytes, or high nibbles), so
//    lane (row j, half h) ends with the exact integer sums n.qh, n.ql of 8 vectors; it then applies
//    the one-vector kernel's fold to each (the same integers ta = sum n q and tb = 16 sum n q, the same
//    float expression), accumulates each group over the super-blocks of each K range of that kernel's
//    geometry (KQ ranges of mx_geometry, walked in its order), and adds the ranges in order, each as
//    (g0 + g2) + (g1 + g3).  An optional bias is added last (out = sum + bias[r], the reference's
//    wmatmulNBias, runtime/include/qorvix/runtime/weights.hpp:68-80).
constexpr int kManyRows = 32;  // weight rows a workgroup

// Also zeroes the ncnt tile counters of the product launch that follows it on the stream.
__global__ __launch_bounds__(256) void k_q4k_many_conv(const float* __restrict__ X, int nvec, int cols,
                                                       uint8_t* __restrict__ frag, float4* __restrict__ meta,
                                                       uint32_t* __restrict__ cnt, int ncnt) {
  const int nsb = cols / 256, per = nsb * 32;
  const int ntask = nvec * per;
  const int t0 = (int)blockIdx.x * 256 + (int)threadIdx.x, t = min(t0, ntask - 1);
  if (t0 < ncnt) cnt[t0] = 0u;
  const int v = t / per, r = t - v * per;
  const float4* src = reinterpret_cast<const float4*>(X + (size_t)v * cols + 8 * r);
  const XQ8 q = mx_quantize(src[0], src[1]);  // every lane takes part: DPP across the 8 tasks of a group
  if (t0 >= ntask) return;
  const int sblk = r >> 5, g = (r >> 3) & 3, part = r & 7;
  const int sb = 2 * g + (part >> 2), off = 8 * (part & 3);
  uint8_t* base = frag + (((size_t)v * nsb + sblk) * 8 + sb) * 64;
  *reinterpret_cast<uint2*>(base + off) = make_uint2(q.h0, q.h1);
  *reinterpret_cast<uint2*>(base + 32 + off) = make_uint2(q.l0, q.l1);
  float* m = reinterpret_cast<float*>(meta + ((size_t)v * nsb + sblk) * 4 + g);
  if (part == 0) {
    m[0] = q.sx;
    m[1] = (float)q.sq;
  }
  if (part == 4) m[2] = (float)q.sq;
}

// Lane (j, h)'s 8 vectors are u = 4 q + 2 h + m (q = 0..3, m = 0..1) of the wave's 16; their records
// sit at 8 h + 2 q + m in the wave's LDS rows, so a lane reads its 8 with two 16-byte reads per field.
__device__ inline int many_pos(int u) { return 8 * ((u >> 1) & 1) + 2 * (u >> 2) + (u & 1); }

typedef int i32x16_t __attribute__((ext_vector_type(16)));

// One super-block's operands for a lane: header, the lane's half of the four groups' code bytes, the A
// fragments of the eight sub-blocks (its row: vector j / 2, qh or ql) and the record it loads for the
// wave.  Loaded one step ahead of use.
struct ManyStep {
  uint4 hd, qv[4], av[8];
  float4 mv;
};

// Launch shape: NVB 16-vector blocks a workgroup (1 or 4), WK waves per block, Z workgroups per tile
// (32 rows x 16 NVB vectors) splitting its K ranges.
struct ManyShape {
  int nvb, wk, z, nvt, nrt, KQ;
};

// Wave wk of split z takes the K ranges kq = z WK + wk, + WK Z, ... (kq < KQ) of the one-vector
// geometry, walking each in that kernel's order.  The ranges' partials are added in range order
// from 0.0f: inside the wave when it takes them all (WK = Z = 1), through LDS when the workgroup's
// waves share them (Z = 1), and through `part` when Z > 1 (NVB = 1): each workgroup stores its
// ranges' partials with device-coherent stores, waits for them, and counts itself in at the tile's
// counter (zeroed by the conversion launch); the last one to arrive reads every range back in order
// and stores the tile -- the protocol of split_k_last.
// PF: load each step's operands one step ahead (more registers, fewer waves a SIMD); without it a
// step's loads are issued at the end of the step before and the other waves cover their latency.
template <bool BIAS, int NVB, int WK, bool PF>
__global__ __launch_bounds__(64 * NVB * WK, PF ? 2 : 3) void k_gemv_q4k_many(
    const uint8_t* __restrict__ W, const uint8_t* __restrict__ frag, const float4* __restrict__ meta,
    float* __restrict__ Y, const float* __restrict__ bias, int rows, int cols, int nvec, uint32_t row_bytes, int KQ,
    int nvt, int Z, float* __restrict__ part, uint32_t* __restrict__ cnt) {
  constexpr int NW = NVB * WK;
  __shared__ __attribute__((aligned(16))) float rec[NW][4][3][16];  // [wave][group][sx, Qa, Qb][position]
  __shared__ __attribute__((aligned(16))) float red[WK > 1 ? NVB * 16 * 64 * 8 : 4];  // [vb][kq][lane][8]
  __shared__ int last;
  const int nsb = cols / 256;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wv = wave % NVB, wk = wave / NVB;  // vector block, K-range phase
  int b = (int)blockIdx.x;
  {
    const int nb = (int)gridDim.x;
    if ((nb & 7) == 0) b = (b & 7) * (nb >> 3) + (b >> 3);  // an XCD takes consecutive tiles: one row block
  }
  const int tile = b / Z, z = b - tile * Z;
  const int rt = tile / nvt, vt = tile - rt * nvt;
  const int j = lane & 31, h = lane >> 5;
  const int r = rt * kManyRows + j, rr = min(r, rows - 1);
  const int vb = vt * 16 * NVB + 16 * wv;
  const uint8_t* wp = W + (size_t)rr * row_bytes;
  const int va = min(vb + (j >> 1), nvec - 1);  // A row j = (vector j / 2, part j % 2)
  const uint8_t* ap = frag + (size_t)va * nsb * 512 + (j & 1) * 32 + 16 * h;
  // record this lane loads for the wave (vector l / 4, group l % 4) and where it goes
  const int mu = lane >> 2, mg = lane & 3;
  const float4* mp = meta + (size_t)min(vb + mu, nvec - 1) * nsb * 4 + mg;
  const uint32_t mw = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) float*)&rec[wave][mg][0][many_pos(mu)];
  const uint32_t mr = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) float*)&rec[wave][0][0][8 * h];
  float* tpart = part + (((size_t)tile * NVB + wv) * KQ) * 512 + lane * 8;  // [kq][lane][8] of this block

  auto load = [&](int sblk, ManyStep& d) {
    const uint8_t* wb = wp + (size_t)sblk * 144;
    d.hd = *reinterpret_cast<const uint4*>(wb);
#pragma unroll
    for (int c = 0; c < 4; ++c) d.qv[c] = *reinterpret_cast<const uint4*>(wb + 16 + 32 * c + 16 * h);
    const uint8_t* fb = ap + (size_t)sblk * 512;
#pragma unroll
    for (int sb = 0; sb < 8; ++sb) d.av[sb] = *reinterpret_cast<const uint4*>(fb + 64 * sb);
    d.mv = mp[(size_t)sblk * 4];
  };
  auto range = [&](int kq, int& s0, int& s1, bool& back) {
    s0 = kq * nsb / KQ;
    s1 = (kq + 1) * nsb / KQ;
    back = KQ > 1 && !(kq & 1);  // SbOrder
  };
  auto sblk_of = [&](int kq, int u) {
    int s0, s1;
    bool back;
    range(kq, s0, s1, back);
    return back ? s1 - 1 - u : s0 + u;
  };
  const int qstep = WK * Z;
  auto advance = [&](int& q, int& uu) {  // next (range, position) of this wave; q >= KQ when done
    int s0, s1;
    bool back;
    range(q, s0, s1, back);
    if (++uu >= s1 - s0) {
      uu = 0;
      for (q += qstep; q < KQ; q += qstep) {
        range(q, s0, s1, back);
        if (s1 > s0) break;
      }
    }
  };
  float fin[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) fin[k] = 0.0f;
  // a range's partial, groups as (g0 + g2) + (g1 + g3)
  auto put = [&](int q, const float (&pk)[8]) {
    if (Z > 1) {
#pragma unroll
      for (int k = 0; k < 8; ++k)
        __hip_atomic_store(tpart + (size_t)q * 512 + k, pk[k], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    } else if constexpr (WK > 1) {
#pragma unroll
      for (int k = 0; k < 8; ++k) red[((wv * KQ + q) * 64 + lane) * 8 + k] = pk[k];
    } else {
#pragma unroll
      for (int k = 0; k < 8; ++k) fin[k] += pk[k];
    }
  };

  const int q0 = z * WK + wk;
  int kq = q0, u = 0;
  {  // skip leading empty ranges
    int s0, s1;
    bool back;
    if (kq < KQ) range(kq, s0, s1, back);
    while (kq < KQ && s1 <= s0) {
      kq += qstep;
      if (kq < KQ) range(kq, s0, s1, back);
    }
  }
  ManyStep cur, nxt;
  if (kq < KQ) load(sblk_of(kq, 0), cur);
  int cur_kq = kq;
  // ranges this wave owns that are empty still contribute (0 + 0) + (0 + 0) = +0 to their slot
  if (Z > 1 || WK > 1) {
    for (int q = q0; q < KQ; q += qstep) {
      int s0, s1;
      bool back;
      range(q, s0, s1, back);
      if (s1 <= s0) {
        const float zero[8] = {};
        put(q, zero);
      }
    }
  }
  float acc[8][4];
#pragma unroll
  for (int k = 0; k < 8; ++k)
#pragma unroll
    for (int c = 0; c < 4; ++c) acc[k][c] = 0.0f;
  while (cur_kq < KQ) {
    int nkq = cur_kq, nu = u;
    advance(nkq, nu);
    if constexpr (PF)
      if (nkq < KQ) load(sblk_of(nkq, nu), nxt);  // next step's operands in flight during this one
    // the wave's records of this super-block into its LDS rows (wave-private: no barrier)
    asm volatile("ds_write_b32 %0, %1 offset:0\n\tds_write_b32 %0, %2 offset:64\n\tds_write_b32 %0, %3 offset:128"
                 ::"v"(mw), "v"(cur.mv.x), "v"(cur.mv.y), "v"(cur.mv.z) : "memory");
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    const u32x4 hd = {cur.hd.x, cur.hd.y, cur.hd.z, cur.hd.w};
    const float d = f16lo(hd.x), dmin = f16hi(hd.x);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const uint4 q = cur.qv[c];
      const v4i bl = {(int)(q.x & 0x0F0F0F0Fu), (int)(q.y & 0x0F0F0F0Fu), (int)(q.z & 0x0F0F0F0Fu),
                      (int)(q.w & 0x0F0F0F0Fu)};
      const v4i bh = {(int)((q.x >> 4) & 0x0F0F0F0Fu), (int)((q.y >> 4) & 0x0F0F0F0Fu),
                      (int)((q.z >> 4) & 0x0F0F0F0Fu), (int)((q.w >> 4) & 0x0F0F0F0Fu)};
      const v4i a0 = __builtin_bit_cast(v4i, cur.av[2 * c]), a1 = __builtin_bit_cast(v4i, cur.av[2 * c + 1]);
      const i32x16_t lo = __builtin_amdgcn_mfma_i32_32x32x32_i8(a0, bl, i32x16_t{}, 0, 0, 0);
      const i32x16_t hi = __builtin_amdgcn_mfma_i32_32x32x32_i8(a1, bh, i32x16_t{}, 0, 0, 0);
      float sca, scb16, mna, mnb;
      q4k_group_scales(hd, c, sca, scb16, mna, mnb);
      // fma((float)(16 S), scb16, p) == fma((float)S, 16 scb16, p): 16 S and 16 scb16 = the 6-bit
      // scale are exact, so both products are the same real and the fma rounds it once
      const float scb = scb16 * 16.0f;
      float sx[8], qa[8], qb[8];
      {
        const uint32_t ra = mr + (uint32_t)c * 192u;
        float4 t0, t1, t2, t3, t4, t5;
        asm volatile("ds_read_b128 %0, %6 offset:0\n\tds_read_b128 %1, %6 offset:16\n\t"
                     "ds_read_b128 %2, %6 offset:64\n\tds_read_b128 %3, %6 offset:80\n\t"
                     "ds_read_b128 %4, %6 offset:128\n\tds_read_b128 %5, %6 offset:144\n\ts_waitcnt lgkmcnt(0)"
                     : "=&v"(t0), "=&v"(t1), "=&v"(t2), "=&v"(t3), "=&v"(t4), "=&v"(t5)
                     : "v"(ra)
                     : "memory");
        const float4 tt[6] = {t0, t1, t2, t3, t4, t5};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          sx[k] = tt[0][k];
          sx[4 + k] = tt[1][k];
          qa[k] = tt[2][k];
          qa[4 + k] = tt[3][k];
          qb[k] = tt[4][k];
          qb[4 + k] = tt[5][k];
        }
      }
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const int e = 4 * (k >> 1) + 2 * (k & 1);  // D rows of vector k: qh at e, ql at e + 1
        const int ta = (int)((uint32_t)lo[e] << 7) + lo[e + 1];                 // sum n q, sub-block 2c
        const int tb = (int)(((uint32_t)hi[e] << 7) + (uint32_t)hi[e + 1]);    // sum n q, 2c + 1
        const float t = __builtin_fmaf((float)tb, scb, (float)ta * sca);
        const float w = __builtin_fmaf(qb[k], mnb, qa[k] * mna);
        acc[k][c] = __builtin_fmaf(__builtin_fmaf(d, t, -dmin * w), sx[k], acc[k][c]);
      }
    }
    if (nkq != cur_kq) {  // the range ends
      float pk[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        pk[k] = (acc[k][0] + acc[k][2]) + (acc[k][1] + acc[k][3]);
#pragma unroll
        for (int c = 0; c < 4; ++c) acc[k][c] = 0.0f;
      }
      put(cur_kq, pk);
    }
    if constexpr (PF)
      cur = nxt;
    else if (nkq < KQ)
      load(sblk_of(nkq, nu), cur);
    cur_kq = nkq;
    u = nu;
  }
  if (Z > 1) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this wave's partial stores have completed
    __syncthreads();
    if (tid == 0)
      last = __hip_atomic_fetch_add(cnt + tile, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == (uint32_t)(Z - 1);
    __syncthreads();
    if (!last || wk != 0) return;
    for (int q = 0; q < KQ; ++q)  // every range in order, as the one-vector kernel adds its waves
#pragma unroll
      for (int k = 0; k < 8; ++k)
        fin[k] += __hip_atomic_load(tpart + (size_t)q * 512 + k, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  } else if constexpr (WK > 1) {
    __syncthreads();
    if (wk != 0) return;
    for (int q = 0; q < KQ; ++q)
#pragma unroll
      for (int k = 0; k < 8; ++k) fin[k] += red[((wv * KQ + q) * 64 + lane) * 8 + k];
  }
  if (r >= rows) return;
  const float bv = BIAS ? bias[r] : 0.0f;
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const int v = vb + 4 * (k >> 1) + 2 * h + (k & 1);
    if (v < nvec) Y[(size_t)v * rows + r] = BIAS ? fin[k] + bv : fin[k];
  }
}

// The launch shape for nvec x rows x cols.  Above 32 vectors, 64 vectors a workgroup (a wave each,
// every K range in the wave: the weights are read once per 64 vectors).  Up to 32, 16 vectors a
// workgroup and one wave per K range (up to 8 a workgroup, the rest split over workgroups), which
// keeps the CUs busy on small batches and on weights of few rows.  Measured on MI355X (Q4_K 14336 x
// 4096, 4096 x 14336, 4096 x 4096, 1024 x 4096): the 16-vector shape is 1.3-3x faster at 16 and 32
// vectors and up to 3x slower from 128 on (it reads the weights once per 16 vectors).
static ManyShape many_shape(int nvec, int rows, int cols, size_t row_bytes) {
  MxGeo geo{};
  (void)mx_geometry(rows, cols, row_bytes, geo);
  ManyShape m{};
  m.KQ = geo.KQ;
  m.nrt = (rows + kManyRows - 1) / kManyRows;
  if (nvec > 32) {
    m.nvb = 4;
    m.wk = 1;
    m.z = 1;
    m.nvt = (nvec + 63) / 64;
  } else {
    m.nvb = 1;
    m.wk = m.KQ < 8 ? m.KQ : 8;
    m.z = m.KQ / m.wk;
    m.nvt = (nvec + 15) / 16;
  }
  return m;
}

// Workspace bytes of a shape: A fragments, records, then (Z > 1) the partials and the tile counters.
static size_t many_ws_bytes(const ManyShape& m, int nvec, int cols) {
  const size_t nsb = (size_t)(cols / 256);
  size_t n = (size_t)nvec * nsb * 512 + (size_t)nvec * nsb * 64;
  if (m.z > 1) n += (size_t)m.nrt * m.nvt * m.nvb * m.KQ * 512 * 4 + (size_t)m.nrt * m.nvt * 4;
  return n;
}

// 1 if the many-vector form takes this call: the shapes the one-vector matrix-core kernel takes (its
// outputs are bit-identical to that kernel's), whole 256-element super-blocks.
int gemv_many_supported(int cols, size_t row_bytes) {
  return gemv_mx_max_nv(cols) >= 1 && row_bytes < (1u << 24) ? 1 : 0;
}

// Workspace bytes of the many-vector form for this call.
size_t gemv_many_ws_bytes(int nvec, int rows, int cols, size_t row_bytes) {
  return many_ws_bytes(many_shape(nvec, rows, cols, row_bytes), nvec, cols);
}

// The many-vector form with a given shape (ws: many_ws_bytes of it, 16-byte aligned).
bool launch_gemv_q4k_many_shape(const void* w, const float* X, float* Y, const float* bias, int nvec, int rows,
                                int cols, size_t row_bytes, void* ws, const ManyShape& m, hipStream_t s) {
  const int nsb = cols / 256;
  auto* frag = static_cast<uint8_t*>(ws);
  auto* meta = reinterpret_cast<float4*>(frag + (size_t)nvec * nsb * 512);
  float* part = reinterpret_cast<float*>(frag + (size_t)nvec * nsb * 576);
  const int ntile = m.nrt * m.nvt;
  uint32_t* cnt = m.z > 1 ? reinterpret_cast<uint32_t*>(part + (size_t)ntile * m.nvb * m.KQ * 512) : nullptr;
  const int ncnt = m.z > 1 ? ntile : 0;
  const size_t ntask = (size_t)nvec * nsb * 32;
  const size_t nthr = ntask > (size_t)ncnt ? ntask : (size_t)ncnt;
  k_q4k_many_conv<<<(unsigned)((nthr + 255) / 256), 256, 0, s>>>(X, nvec, cols, frag, meta, cnt, ncnt);
  const unsigned grid = (unsigned)((int64_t)ntile * m.z);
  const unsigned thr = (unsigned)(64 * m.nvb * m.wk);
  const auto* wb = static_cast<const uint8_t*>(w);
  const uint32_t rb = (uint32_t)row_bytes;
#define QVX_MANY(B, N, K, P)                                                                                  \
  k_gemv_q4k_many<B, N, K, P><<<grid, thr, 0, s>>>(wb, frag, meta, Y, bias, rows, cols, nvec, rb, m.KQ, m.nvt, \
                                                   m.z, part, cnt)
#define QVX_MANY_WK(B)                          \
  switch (m.wk) {                               \
    case 1: QVX_MANY(B, 1, 1, true); break;     \
    case 2: QVX_MANY(B, 1, 2, true); break;     \
    case 4: QVX_MANY(B, 1, 4, true); break;     \
    default: QVX_MANY(B, 1, 8, true); break;    \
  }
  if (m.nvb == 4) {
    if (bias) QVX_MANY(true, 4, 1, false);
    else QVX_MANY(false, 4, 1, false);
  } else if (bias) {
    QVX_MANY_WK(true)
  } else {
    QVX_MANY_WK(false)
  }
#undef QVX_MANY_WK
#undef QVX_MANY
  return true;
}

// ---- batched Q4_K with the K range split over workgroups -------------------------------------------
// qvx_qmatmul_n over Q4_K, NV (8 or 16) vectors a launch, each weight byte streamed once, every output
// bit-identical to the one-vector kernel's (k_gemv_mx): the many-vector form's arithmetic per group
// (the same MFMA sums, the same fold), the same chains and the same order of the K ranges.
//  * Columns: RPC consecutive whole K ranges of mx_geometry (C super-blocks, at most 8), so every
//    range's chain stays in one workgroup.  Workgroup b (16 waves) owns column b % ncol and the
//    32-row tiles b / ncol, b / ncol + P, ...  Its items are the column's (super-block, group) pairs,
//    item i = 4 sbl + c, taken by wave i % 16 (one or two a wave).  A wave's A fragments (sub-blocks
//    2c and 2c + 1, 16 vectors x qh / ql) are the same for every tile: converted once (mx_quantize,
//    through LDS, into registers); the records (Qa, Qb for the fold, sx for the chains) stay in LDS.
//  * Tiles stream through a two-stage LDS ring (32 rows x the column's bytes, copied by
//    buffer_load_dword ... lds, rows an odd number of dwords apart).  Per tile and item the wave runs
//    the group's two v_mfma_i32_32x32x32_i8 and the fold V = fma(d, t, -dmin w) per (row, vector)
//    into LDS; then four threads an output (one a group) run each range's chain A_c = fma(V, sx, A_c)
//    over its super-blocks in the one-vector kernel's walk order (SbOrder) and add (A0 + A2) +
//    (A1 + A3) across the quad: the range's partial, stored to the workspace.
//  * k_q4s_sum adds each output's KQ range partials in order from 0.0f, then the bias.
struct Q4sGeo {
  int nsb;     // super-blocks a row
  int KQ;      // K ranges of the one-vector geometry
  int RPC;     // ranges a column
  int ncol;    // columns (KQ / RPC)
  int ntile;   // 32-row tiles
  int P;       // workgroups a column
  int C;       // super-blocks of the widest column (<= 4 IPW)
  uint32_t row_bytes;
};

// The range kq's super-blocks [s0, s1) and walk direction (SbOrder: even ranges backward).
__device__ __host__ inline void q4s_range(int kq, int nsb, int KQ, int& s0, int& s1, bool& back) {
  s0 = kq * nsb / KQ;
  s1 = (kq + 1) * nsb / KQ;
  back = KQ > 1 && !(kq & 1);
}

// A 16-byte global load whose wait the kernel places itself (q4s_wait_x), before tile 0's copies:
// the compiler, which does not see those, would otherwise wait for them too at the value's first use.
typedef float q4s_f4 __attribute__((ext_vector_type(4)));
__device__ inline q4s_f4 q4s_ldx(const float* p) {
  q4s_f4 r;
  asm volatile("global_load_dwordx4 %0, %1, off" : "=v"(r) : "v"(p));
  return r;
}
// Waits until at most N vector memory operations are outstanding; the loaded values are operands,
// so no use of them moves above the wait.
template <int N, int K>
__device__ inline void q4s_wait_x(q4s_f4* a, q4s_f4* b) {
  if constexpr (K == 1)
    asm volatile("s_waitcnt vmcnt(%2)" : "+v"(a[0]), "+v"(b[0]) : "n"(N) : "memory");
  else if constexpr (K == 2)
    asm volatile("s_waitcnt vmcnt(%4)" : "+v"(a[0]), "+v"(a[1]), "+v"(b[0]), "+v"(b[1]) : "n"(N) : "memory");
  else
    asm volatile("s_waitcnt vmcnt(%8)"
                 : "+v"(a[0]), "+v"(a[1]), "+v"(a[2]), "+v"(a[3]), "+v"(b[0]), "+v"(b[1]), "+v"(b[2]), "+v"(b[3])
                 : "n"(N)
                 : "memory");
}
// s_waitcnt vmcnt(0) that memory accesses cannot move across.
__device__ inline void q4s_wait_vm0() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }
// Workgroup barrier for LDS only (see q6s_lds_barrier).
__device__ inline void q4s_lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }
// Copy global -> LDS, 4 bytes a lane, as inline asm (see q6s_copy4: the kernel waits for its copies
// itself; the s_nop is the wait state between the M0 write and the copy).
__device__ inline void q4s_copy4(__amdgpu_buffer_rsrc_t r, uint32_t dst, uint32_t voff, uint32_t soff) {
  asm volatile("s_nop 0\n\tbuffer_load_dword %0, %1, %2 offen lds" ::"v"(voff), "s"(r), "s"(soff), "{m0}"(dst)
               : "memory");
}

// s_waitcnt vmcnt(N) for the N = 0..3 tiles' copies that may stay in flight.
template <int CPT>
__device__ inline void q4s_wait_tiles(int n) {
  switch (n) {
    case 0: asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); break;
    case 1: asm volatile("s_waitcnt vmcnt(%0)" ::"n"(CPT) : "memory"); break;
    case 2: asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * CPT) : "memory"); break;
    default: asm volatile("s_waitcnt vmcnt(%0)" ::"n"(3 * CPT) : "memory"); break;
  }
}

// LDS plan of a launch: WPC workgroups a CU.  With one, whole 64-dword copies (every wave makes CPT a
// tile, so the waits can count them) into up to 4 ring stages; with two (8 vectors, one item a wave),
// the copies stop at the column's end and the ring has 2 stages.
template <int NV, int IPW, int WPC>
struct Q4sLds {
  static constexpr int CMAX = 4 * IPW;                  // super-blocks a column at most
  static constexpr int NIT = 4 * CMAX;                  // items at most
  static constexpr int NO = NV * 32;                    // outputs a tile
  static constexpr int NCP = (36 * CMAX + 63) / 64;     // 64-dword copies a staged row
  static constexpr int CPT = 2 * NCP;                   // copies a wave a tile
  static constexpr int SW = (WPC == 1 ? 64 * NCP : 36 * CMAX) + 1;  // LDS dwords a staged row (odd: rows on distinct banks)
  static constexpr int STAGE = 32 * SW * 4;             // bytes of a ring stage
  static constexpr int RB = NV == 8 && IPW == 1 ? 2 : 1;  // step-value buffers
  static constexpr int RES = NIT * NO * 4;              // bytes of one
  static constexpr int BUDGET = 160 * 1024 / WPC - NIT * 3 * 16 * 4 - 64;  // the CU's share less recq, sxl
  static constexpr int NSF = (BUDGET - RB * RES) / STAGE;
  static constexpr int NS = WPC == 2 ? 2 : NSF > 4 ? 4 : NSF;  // ring stages
  static constexpr int BYTES = NS * STAGE + RB * RES;
  static_assert(NS >= 2 && BYTES <= BUDGET, "two ring stages at least, within the budget");
  static_assert(NV * CMAX * 512 <= STAGE + RB * RES, "conversion scratch fits in the last stage + the buffers");
};

template <int NV, int IPW, int WPC>
__global__ __launch_bounds__(1024, 4 * WPC) void k_gemv_q4s(const uint8_t* __restrict__ W, const float* __restrict__ X,
                                                            int rows, int cols, int nv, Q4sGeo geo,
                                                            float* __restrict__ part) {
  static_assert(NV == 8 || NV == 16, "8 or 16 vectors a launch");
  static_assert(IPW == 1 || IPW == 2, "one or two items a wave");
  static_assert(WPC == 1 || (WPC == 2 && NV == 8 && IPW == 1), "two workgroups a CU: 8 vectors, one item a wave");
  using L = Q4sLds<NV, IPW, WPC>;
  constexpr int NIT = L::NIT, NO = L::NO, NCP = L::NCP, SW = L::SW, STAGE = L::STAGE, RB = L::RB, NS = L::NS;
  constexpr int KV = NV / 2;  // vectors a lane folds
  __shared__ __attribute__((aligned(16))) uint8_t lds[L::BYTES];
  __shared__ __attribute__((aligned(16))) float recq[NIT][2][16];  // [item][Qa, Qb][vector]
  __shared__ float sxl[NIT][NV];                                    // [item][vector]
  float* res = reinterpret_cast<float*>(lds + NS * STAGE);          // [buffer][item][vector][row]
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int j = lane & 31, h = lane >> 5;
  const int col = (int)blockIdx.x % geo.ncol, pi = (int)blockIdx.x / geo.ncol;
  const int ntl = pi < geo.ntile ? (geo.ntile - pi + geo.P - 1) / geo.P : 0;
  if (ntl == 0) return;  // the whole workgroup
  int cs0, cs1;          // the column's super-blocks
  {
    bool bk;
    int t0, t1;
    q4s_range(col * geo.RPC, geo.nsb, geo.KQ, cs0, t0, bk);
    q4s_range(col * geo.RPC + geo.RPC - 1, geo.nsb, geo.KQ, t1, cs1, bk);
  }
  const int C = cs1 - cs0, nit = 4 * C;
  const uint32_t lds_base = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(QVX_LDS uint8_t*)lds);

  // Copy of the workgroup's jt-th tile into stage s: wave w copies rows 2w, 2w + 1 (rows past the
  // weight repeat its last row), each as NCP copies of 64 dwords from the column's first byte on --
  // whole ones with one workgroup a CU (past the column: the row's next bytes, or zeros past the
  // weight: the buffer's range; every offset is in the checked vector offset), so that every wave
  // makes CPT copies a tile and the waits can count them; with two, up to the column's end.
  auto issue = [&](int jt, int s) __attribute__((always_inline)) {
    const int r0 = (pi + jt * geo.P) * 32, nr = min(32, rows - r0);
    const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(W + (size_t)r0 * geo.row_bytes), (short)0, (int)((uint32_t)nr * geo.row_bytes), (int)kRsrcWord3);
#pragma unroll
    for (int rr = 0; rr < 2; ++rr) {
      const int r = min(2 * wave + rr, nr - 1);
      const uint32_t vo = (uint32_t)r * geo.row_bytes + (uint32_t)cs0 * 144u + 4u * lane;
      const uint32_t dst = lds_base + (uint32_t)(s * STAGE + (2 * wave + rr) * SW * 4);
#pragma unroll
      for (int i = 0; i < NCP; ++i)
        if (WPC == 1 || 64 * i + lane < 36 * C) q4s_copy4(rsrc, dst + 256u * i, vo + 256u * i, 0u);
    }
  };

  // The activations of the column, every vector, converted once into the last stage + the buffers
  // (not in use yet) in the many-vector layout -- A fragments [v][sbl][sub-block][qh / ql][32 bytes]
  // -- and the records into recq / sxl.  Tiles 0..NS-2 are copied during the conversion.
  constexpr int NTK = NV * L::CMAX * 32 / 1024;  // conversion tasks a thread at most
  static_assert(NTK == 1 || NTK == 2 || NTK == 4, "one, two or four conversion tasks a thread");
  uint8_t* fr = lds + (NS - 1) * STAGE;
  {
    q4s_f4 y0[NTK], y1[NTK];
#pragma unroll
    for (int k = 0; k < NTK; ++k) {
      const int t = min(tid + 1024 * k, NV * C * 32 - 1);
      const int v = t / (C * 32), r = t - v * C * 32;  // r: task of the column, 8 elements
      const float* src = X + (size_t)min(v, nv - 1) * cols + (size_t)cs0 * 256 + 8 * r;
      y0[k] = q4s_ldx(src);
      y1[k] = q4s_ldx(src + 4);
    }
    q4s_wait_x<0, NTK>(y0, y1);
    for (int jt = 0; jt < NS - 1 && jt < ntl; ++jt) issue(jt, jt);
#pragma unroll
    for (int k = 0; k < NTK; ++k) {
      if (1024 * k + 64 * wave >= NV * C * 32) break;  // wave-uniform: no task left for this wave
      const int T = tid + 1024 * k, t = min(T, NV * C * 32 - 1);
      const int v = t / (C * 32), r = t - v * C * 32;
      const bool pad = v >= nv;  // padding vectors: zero fragments and records
      const float4 x0 = pad ? make_float4(0.0f, 0.0f, 0.0f, 0.0f) : make_float4(y0[k].x, y0[k].y, y0[k].z, y0[k].w);
      const float4 x1 = pad ? make_float4(0.0f, 0.0f, 0.0f, 0.0f) : make_float4(y1[k].x, y1[k].y, y1[k].z, y1[k].w);
      const XQ8 q = mx_quantize(x0, x1);  // every lane of the wave takes part
      if (T < NV * C * 32) {
        const int sbl = r >> 5, g = (r >> 3) & 3, pt = r & 7;
        const int sub = 2 * g + (pt >> 2), off = 8 * (pt & 3);
        uint8_t* base = fr + ((v * C + sbl) * 8 + sub) * 64;
        *reinterpret_cast<uint2*>(base + off) = make_uint2(q.h0, q.h1);
        *reinterpret_cast<uint2*>(base + 32 + off) = make_uint2(q.l0, q.l1);
        const int it = 4 * sbl + g;
        if (pt == 0) {
          sxl[it][v] = q.sx;
          recq[it][0][v] = (float)q.sq;
        }
        if (pt == 4) recq[it][1][v] = (float)q.sq;
      }
    }
  }
  q4s_lds_barrier();
  // a wave's A fragments: lane (row j = (vector j / 2, part j % 2), K half h) of sub-blocks 2c, 2c + 1
  v4i af[IPW][2];
#pragma unroll
  for (int i = 0; i < IPW; ++i) {
    const int it = wave + 16 * i, sbl = it >> 2, c = it & 3, va = j >> 1;
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const bool on = it < nit && va < NV;
      const uint8_t* p = fr + ((min(va, NV - 1) * C + min(sbl, C - 1)) * 8 + 2 * c + e) * 64 + (j & 1) * 32 + 16 * h;
      const v4i z = {0, 0, 0, 0};
      af[i][e] = on ? *reinterpret_cast<const v4i*>(p) : z;
    }
  }
  q4s_lds_barrier();  // every wave's fragments are in registers: the last stage and the buffers are free

  auto fold = [&](int s, float* rb) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < IPW; ++i) {
      const int it = wave + 16 * i;
      if (it >= nit) break;  // wave-uniform
      const int sbl = it >> 2, c = it & 3;
      const uint8_t* rowp = lds + s * STAGE + j * SW * 4 + sbl * 144;
      const uint32_t* hp = reinterpret_cast<const uint32_t*>(rowp);
      const uint32_t* qp = reinterpret_cast<const uint32_t*>(rowp + 16 + 32 * c + 16 * h);
      const u32x4 hd = {hp[0], hp[1], hp[2], hp[3]};
      const uint32_t q0 = qp[0], q1 = qp[1], q2 = qp[2], q3 = qp[3];
      const v4i bl = {(int)(q0 & 0x0F0F0F0Fu), (int)(q1 & 0x0F0F0F0Fu), (int)(q2 & 0x0F0F0F0Fu), (int)(q3 & 0x0F0F0F0Fu)};
      const v4i bh = {(int)((q0 >> 4) & 0x0F0F0F0Fu), (int)((q1 >> 4) & 0x0F0F0F0Fu), (int)((q2 >> 4) & 0x0F0F0F0Fu),
                      (int)((q3 >> 4) & 0x0F0F0F0Fu)};
      const i32x16_t lo = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[i][0], bl, i32x16_t{}, 0, 0, 0);
      const i32x16_t hi = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[i][1], bh, i32x16_t{}, 0, 0, 0);
      const float d = f16lo(hd.x), dmin = f16hi(hd.x);
      float sca, scb16, mna, mnb;
      q4k_group_scales(hd, c, sca, scb16, mna, mnb);
      const float scb = scb16 * 16.0f;  // see the many-vector form: the same product, rounded once
#pragma unroll
      for (int k = 0; k < KV; ++k) {
        const int e = 4 * (k >> 1) + 2 * (k & 1), v = 4 * (k >> 1) + 2 * h + (k & 1);
        const int ta = (int)((uint32_t)lo[e] << 7) + lo[e + 1];
        const int tb = (int)(((uint32_t)hi[e] << 7) + (uint32_t)hi[e + 1]);
        const float t = __builtin_fmaf((float)tb, scb, (float)ta * sca);
        const float w = __builtin_fmaf(recq[it][1][v], mnb, recq[it][0][v] * mna);
        rb[(it * NV + v) * 32 + j] = __builtin_fmaf(d, t, -dmin * w);
      }
    }
  };
  auto chains = [&](int jt, const float* rb) __attribute__((always_inline)) {
    const int tile = pi + jt * geo.P;
#pragma unroll
    for (int o4 = tid; o4 < 4 * NO; o4 += 1024) {
      const int o = o4 >> 2, c = o4 & 3, v = o >> 5;
      for (int q = 0; q < geo.RPC; ++q) {
        const int kq = col * geo.RPC + q;
        int s0, s1;
        bool back;
        q4s_range(kq, geo.nsb, geo.KQ, s0, s1, back);
        float A = 0.0f;
        for (int u = 0; u < s1 - s0; ++u) {
          const int it = 4 * ((back ? s1 - 1 - u : s0 + u) - cs0) + c;
          A = __builtin_fmaf(rb[it * NO + o], sxl[it][v], A);
        }
        float u2 = A + dppf<0x4E>(A);  // quad_perm [2,3,0,1]: (A0 + A2) on the quad's lanes 0, 2, (A1 + A3) on 1, 3
        u2 = u2 + dppf<0xB1>(u2);      // quad_perm [1,0,3,2]: (A0 + A2) + (A1 + A3)
        if (c == 0) part[((size_t)tile * geo.KQ + kq) * NO + o] = u2;
      }
    }
  };

  // Tile jt: wait for its copies (up to NS - 2 later tiles' may stay in flight), then, after the
  // barrier, copy tile jt + NS - 1 into the stage of tile jt - 1 (read by every wave by now), fold
  // tile jt into the step values, and form the range partials (8 vectors, one item a wave: of tile
  // jt - 1 from the other buffer; else of tile jt after a second barrier).
  for (int jt = 0; jt < ntl; ++jt) {
    const int s = jt % NS;
    if constexpr (NS == 2)
      q4s_wait_vm0();
    else
      q4s_wait_tiles<L::CPT>(min(NS - 2, ntl - 1 - jt));
    q4s_lds_barrier();
    if (jt + NS - 1 < ntl) issue(jt + NS - 1, (jt + NS - 1) % NS);
    if constexpr (RB == 2) {
      if (jt > 0) chains(jt - 1, res + ((jt - 1) & 1) * (L::RES / 4));
      fold(s, res + (jt & 1) * (L::RES / 4));
    } else {
      fold(s, res);
      q4s_lds_barrier();
      chains(jt, res);
    }
  }
  if constexpr (RB == 2) {
    q4s_lds_barrier();
    chains(ntl - 1, res + ((ntl - 1) & 1) * (L::RES / 4));
  }
}

// out[v, r] = the KQ range partials of (v, r) added in order from 0.0f (+ bias[r]).
template <bool BIAS>
__global__ __launch_bounds__(256) void k_q4s_sum(const float* __restrict__ part, float* __restrict__ Y,
                                                 const float* __restrict__ bias, int rows, int nv, int KQ, int NO,
                                                 int ntile) {
  const int idx = (int)blockIdx.x * 256 + (int)threadIdx.x;
  if (idx >= ntile * NO) return;
  const int tile = idx / NO, o = idx - tile * NO, v = o >> 5, r = tile * 32 + (o & 31);
  if (v >= nv || r >= rows) return;
  const float* p = part + (size_t)tile * KQ * NO + o;
  float sum = 0.0f;
  for (int k0 = 0; k0 < KQ; k0 += 8) {  // eight partials in flight at a time, added in order
    float b8[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) b8[k] = p[(size_t)min(k0 + k, KQ - 1) * NO];
#pragma unroll
    for (int k = 0; k < 8; ++k)
      if (k0 + k < KQ) sum += b8[k];
  }
  Y[(size_t)v * rows + r] = BIAS ? sum + bias[r] : sum;
}

int device_cus();

// The launch geometry: the one-vector geometry's ranges grouped into columns of >= 4 super-blocks
// where they can be (and <= 8); false when a range alone is wider than 8 super-blocks.
static bool q4s_geometry(int rows, int cols, size_t row_bytes, Q4sGeo& g) {
  if (gemv_many_supported(cols, row_bytes) == 0 || rows <= 0) return false;
  MxGeo mg{};
  (void)mx_geometry(rows, cols, row_bytes, mg);
  g.nsb = cols / 256;
  g.KQ = mg.KQ;
  g.ntile = (rows + 31) / 32;
  g.row_bytes = (uint32_t)row_bytes;
  auto width = [&](int rpc) {  // widest column of rpc ranges
    int w = 0;
    for (int c0 = 0; c0 < g.KQ; c0 += rpc) {
      int s0, s1, t0, t1;
      bool b;
      q4s_range(c0, g.nsb, g.KQ, s0, t0, b);
      q4s_range(c0 + rpc - 1, g.nsb, g.KQ, t1, s1, b);
      w = std::max(w, s1 - s0);
    }
    return w;
  };
  g.RPC = 0;
  for (int r = 1; r <= g.KQ; ++r) {
    if (g.KQ % r) continue;
    const int w = width(r);
    if (w > 8) break;
    g.RPC = r;
    g.C = w;
    int lo = g.nsb;  // narrowest column
    for (int c0 = 0; c0 < g.KQ; c0 += r) {
      int s0, s1, t0, t1;
      bool b;
      q4s_range(c0, g.nsb, g.KQ, s0, t0, b);
      q4s_range(c0 + r - 1, g.nsb, g.KQ, t1, s1, b);
      lo = std::min(lo, s1 - s0);
    }
    if (lo >= 4) break;
  }
  if (g.RPC == 0) return false;
  g.ncol = g.KQ / g.RPC;
  g.P = std::max(1, std::min(g.ntile, device_cus() / g.ncol));
  return true;
}

// 1 if the split Q4_K form takes the shape, and its workspace bytes for nvec vectors (the range
// partials) through *ws_bytes.
bool gemv_q4s_route(int nvec, int rows, int cols, size_t row_bytes, size_t* ws_bytes) {
  Q4sGeo g;
  if (nvec <= 0 || !q4s_geometry(rows, cols, row_bytes, g)) return false;
  if (ws_bytes) *ws_bytes = (size_t)g.ntile * g.KQ * (nvec <= 8 ? 8 : 16) * 32 * 4;
  return true;
}

// qmatmul_n over Q4_K on the split form, 16 vectors a launch (8 when the whole call has at most 8),
// each launch followed by the in-order sum of its range partials (and the bias).
bool launch_gemv_q4s(const void* w, const float* X, float* Y, const float* bias, int nvec, int rows, int cols,
                     size_t row_bytes, void* ws, hipStream_t s) {
  Q4sGeo g;
  if (nvec <= 0 || !ws || !q4s_geometry(rows, cols, row_bytes, g)) return false;
  const int nvp = nvec <= 8 ? 8 : 16, NO = nvp * 32;
  const auto* wb = static_cast<const uint8_t*>(w);
  auto* part = static_cast<float*>(ws);
  const unsigned grid = (unsigned)(g.ncol * g.P);
  const bool ipw2 = g.C > 4;
  for (int v0 = 0; v0 < nvec; v0 += nvp) {
    const int nv = std::min(nvp, nvec - v0);
    const float* Xv = X + (size_t)v0 * cols;
    float* Yv = Y + (size_t)v0 * rows;
    if (nvp == 8 && !ipw2) {
      const int P2 = std::max(1, std::min(g.ntile, 2 * device_cus() / g.ncol));
      Q4sGeo g2 = g;
      g2.P = P2;
      k_gemv_q4s<8, 1, 2><<<(unsigned)(g.ncol * P2), 1024, 0, s>>>(wb, Xv, rows, cols, nv, g2, part);
    } else if (nvp == 8) {
      k_gemv_q4s<8, 2, 1><<<grid, 1024, 0, s>>>(wb, Xv, rows, cols, nv, g, part);
    } else {
      if (ipw2) k_gemv_q4s<16, 2, 1><<<grid, 1024, 0, s>>>(wb, Xv, rows, cols, nv, g, part);
      else k_gemv_q4s<16, 1, 1><<<grid, 1024, 0, s>>>(wb, Xv, rows, cols, nv, g, part);
    }
    const unsigned sg = (unsigned)((g.ntile * NO + 255) / 256);
    if (bias) k_q4s_sum<true><<<sg, 256, 0, s>>>(part, Yv, bias, rows, nv, g.KQ, NO, g.ntile);
    else k_q4s_sum<false><<<sg, 256, 0, s>>>(part, Yv, nullptr, rows, nv, g.KQ, NO, g.ntile);
  }
  return true;
}

// Q4_K GEMV of nvec vectors with the activations converted once (bias may be null).  ws: the
// gemv_many_ws_bytes workspace, 16-byte aligned.  Returns false, having launched nothing, when the
// shape is not handled here.
bool launch_gemv_q4k_many(const void* w, const float* X, float* Y, const float* bias, int nvec, int rows, int cols,
                          size_t row_bytes, void* ws, hipStream_t s) {
  if (!gemv_many_supported(cols, row_bytes) || nvec < 1 || rows < 1 || !ws) return false;
  return launch_gemv_q4k_many_shape(w, X, Y, bias, nvec, rows, cols, row_bytes, ws,
                                    many_shape(nvec, rows, cols, row_bytes), s);
}

}  // namespace qvx
