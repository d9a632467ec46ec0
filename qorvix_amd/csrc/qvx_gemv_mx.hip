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
//    These 16-byte fragments are built once per workgroup in LDS, in MFMA order.
//  * After the 4 MFMAs the accumulator of lane (j, c) holds rows 4c..4c+3 of column j, i.e. the
//    four partial sums (lo.qh, lo.ql, hi.qh, hi.ql) of row j over group c: the lane applies the
//    group's scale/min fold exactly as the VALU kernel does.  K positions are matched between A
//    and B lane by lane and register by register, so the product does not depend on how the
//    instruction orders K inside a lane group.
//
// Data movement: each wave owns a ring of NB LDS stages.  A tile's 2304 bytes (16 rows x 144) are
// copied with three buffer_load_dwordx4 ... lds (chunk q = 64k + lane -> row q/9, 16-byte chunk
// q%9, LDS offset 16q: rows 144 bytes apart, conflict-free for the 16-lane quarter reads; the
// super-block offset is the scalar soffset), NB-1 tiles ahead of use; the wave waits for a tile with
// s_waitcnt vmcnt (the copies are its only vector memory operations in the loop) and reads it back
// in MFMA order.  The loop reads LDS through inline asm (see lds_read16).
//
// Work: workgroup b owns rows [rb, rb + cnt) (cnt <= 16 TQ); wave w = kq * TQ + tq takes tile tq
// and super-blocks [kq nsb / KQ, (kq + 1) nsb / KQ).  Per-lane partials are summed over the four
// groups with permlane swaps and over the KQ waves of a tile in wave order through LDS, so every
// output's arithmetic is fixed: one vector's result does not depend on the other vectors of the
// launch, and qvx_qmatmul_n stays bit-identical to qvx_qmatmul per vector.
#include <algorithm>

#include "qvx_common.hpp"

namespace qvx {

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef short short2_t __attribute__((ext_vector_type(2)));
#define QVX_LDS __attribute__((address_space(3)))

constexpr int kSB = 144;          // Q4_K super-block bytes
constexpr int kTileBytes = 2304;  // 16 rows x one super-block
constexpr int kFragBytes = 1024;  // A fragments of one (vector, super-block): [group][part][m] x 16 bytes
constexpr uint32_t kRsrcWord3 = 0x00020000u;  // raw buffer, 32-bit data (gfx9)

struct MxGeo {
  int nsb;        // super-blocks per row
  int base, rem;  // workgroup b owns base + (b < rem) rows starting at b*base + min(b, rem)
  int TQ, KQ;     // tiles per workgroup, K splits; TQ * KQ = 16 waves
  uint32_t row_bytes;
};

// LDS: dynamic [fragments: NV*nsb*1024][meta: NV*nsb*4 groups*16][zero: 64] and a static tile ring
// [16 waves][NB][2304].
__host__ __device__ inline size_t mx_frag_bytes(int nv, int nsb) { return (size_t)nv * nsb * kFragBytes; }
__host__ __device__ inline size_t mx_meta_bytes(int nv, int nsb) { return (size_t)nv * nsb * 4 * 16; }
__host__ __device__ inline size_t mx_dyn_bytes(int nv, int nsb) { return mx_frag_bytes(nv, nsb) + mx_meta_bytes(nv, nsb) + 64; }
__host__ __device__ inline size_t mx_lds_bytes(int nv, int nsb, int nb) {
  return mx_dyn_bytes(nv, nsb) + (size_t)16 * nb * kTileBytes;
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
__device__ inline void lds_wait(u32x4& a, u32x4& b, u32x4& c, u32x4& d, u32x4& e) {
  asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(a), "+v"(b), "+v"(c), "+v"(d), "+v"(e)::"memory");
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

__device__ inline void mx_convert(const float4 x0, const float4 x1, int v, int sg, int part, bool store,
                                  uint8_t* frag, float* meta, int nsb) {
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
  if (store) {
    const uint32_t h0 = __builtin_amdgcn_perm(hs[1], hs[0], 0x06040200u), h1 = __builtin_amdgcn_perm(hs[3], hs[2], 0x06040200u);
    const uint32_t l0 = __builtin_amdgcn_perm(ls[1], ls[0], 0x06040200u), l1 = __builtin_amdgcn_perm(ls[3], ls[2], 0x06040200u);
    const int g = sg & 3, s = sg >> 2, hi = part >> 2, m = part & 3;
    uint8_t* f = frag + (size_t)(v * nsb + s) * kFragBytes + g * 256 + 2 * hi * 64 + m * 16;  // parts 2hi, 2hi+1
    const uint4 fh = hi ? make_uint4(0u, 0u, h0, h1) : make_uint4(h0, h1, 0u, 0u);
    const uint4 fl = hi ? make_uint4(0u, 0u, l0, l1) : make_uint4(l0, l1, 0u, 0u);
    *reinterpret_cast<uint4*>(f) = fh;
    *reinterpret_cast<uint4*>(f + 64) = fl;
    float* mt = meta + ((size_t)(v * nsb + s) * 4 + g) * 4;  // [sx, Qa, Qb, 128 Qb as int]
    if (part == 0) {
      mt[0] = a * (1.0f / 16383.0f) + z;
      mt[1] = (float)sq;
    }
    if (part == 4) {
      mt[2] = (float)sq;
      mt[3] = __builtin_bit_cast(float, 128 * sq);
    }
  }
}

// Copy a tile (16 rows of this wave, super-block s) into an LDS stage: chunk q = 64k + lane.
__device__ inline void mx_issue(__amdgpu_buffer_rsrc_t rsrc, const uint32_t (&off)[3], int s, QVX_LDS uint8_t* st,
                                int lane) {
  const uint32_t so = (uint32_t)s * kSB;
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, st, 16, off[0], so, 0, 0);
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, st + 1024, 16, off[1], so, 0, 0);
  if (lane < 16) __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, st + 2048, 16, off[2], so, 0, 0);
}

template <int NV, int NB, int TPT>
__global__ __launch_bounds__(1024) void k_gemv_mx(const uint8_t* __restrict__ W, const float* __restrict__ X,
                                                  float* __restrict__ Y, int rows, int cols, MxGeo geo) {
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  __shared__ __attribute__((aligned(16))) uint8_t ring[16 * NB * kTileBytes];
  const int nsb = geo.nsb, TQ = geo.TQ, KQ = geo.KQ;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: scalar offsets, M0
  uint8_t* frag = lds;
  float* meta = reinterpret_cast<float*>(lds + mx_frag_bytes(NV, nsb));
  uint8_t* zero = lds + mx_frag_bytes(NV, nsb) + mx_meta_bytes(NV, nsb);
  QVX_LDS uint8_t* stage = (QVX_LDS uint8_t*)(ring + wave * NB * kTileBytes);

  const int b = blockIdx.x;
  const int rb = b * geo.base + min(b, geo.rem), cnt = geo.base + (b < geo.rem ? 1 : 0);
  const int tq = wave % TQ, kq = wave / TQ;
  const int s0 = kq * nsb / KQ, s1 = (kq + 1) * nsb / KQ, nu = s1 - s0;

  // 1. this thread's activations (requested first: vector loads complete in order)
  const int per = nsb * 32, ntask = NV * per;
  float4 xr[TPT][2];
#pragma unroll
  for (int k = 0; k < TPT; ++k) {
    const int t = min(tid + 1024 * k, ntask - 1), v = task_vec<NV>(t, per), r = t - v * per;
    const float4* src = reinterpret_cast<const float4*>(X + (size_t)v * cols + 8 * r);
    xr[k][0] = src[0];
    xr[k][1] = src[1];
  }

  // 2. A fragments into LDS (waves without tasks skip)
#pragma unroll
  for (int k = 0; k < TPT; ++k) {
    if (1024 * k + 64 * wave < ntask) {
      const int t0 = tid + 1024 * k, t = min(t0, ntask - 1), v = task_vec<NV>(t, per), r = t - v * per;
      mx_convert(xr[k][0], xr[k][1], v, r >> 3, r & 7, t0 < ntask, frag, meta, nsb);
    }
  }
  if (tid < 16) reinterpret_cast<uint32_t*>(zero)[tid] = 0u;

  // 3. prologue copies (tiles of the first NB-1 super-blocks; rows past cnt read as zeros), issued
  // after the activations are consumed so no compiler-inserted wait covers them
  const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(W + (size_t)rb * geo.row_bytes), (short)0, (int)((uint32_t)cnt * geo.row_bytes), (int)kRsrcWord3);
  uint32_t off[3];
#pragma unroll
  for (int k = 0; k < 3; ++k) {
    const uint32_t q = (uint32_t)min(64 * k + lane, 143), r = q / 9u, c9 = q - 9u * r;
    off[k] = __umul24(16u * (uint32_t)tq + r, geo.row_bytes) + 16u * c9;
  }
#pragma unroll
  for (int u = 0; u < NB - 1; ++u) mx_issue(rsrc, off, min(s0 + u, nsb - 1), stage + u * kTileBytes, lane);

  // Barrier for the fragments only: wait for this wave's LDS writes, not for the tile copies in
  // flight (__syncthreads would wait for those too).
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
  __builtin_amdgcn_s_barrier();

  // 4. tiles
  const int j = lane & 15, g = lane >> 4;  // B column (tile row) / K block = group; A row = j
  const uint32_t b_hd = kSB * j, b_q = kSB * j + 16 + 32 * g;
  const bool aon = (j >> 2) == g;
  const uint32_t a_rel = (uint32_t)(g * 256 + (j & 3) * 64);
  const uint32_t frag_base = (uint32_t)(uintptr_t)(QVX_LDS uint8_t*)frag;
  const uint32_t meta_base = (uint32_t)(uintptr_t)(QVX_LDS uint8_t*)meta + 16u * g;
  const uint32_t zero_base = (uint32_t)(uintptr_t)(QVX_LDS uint8_t*)zero;
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
  for (int u = 0; u < nu; ++u) {
    if (u + NB - 1 < nu) {
      const int ns = slot + NB - 1 >= NB ? slot - 1 : slot + NB - 1;  // (slot + NB - 1) % NB
      mx_issue(rsrc, off, s0 + u + NB - 1, stage + ns * kTileBytes, lane);
      wait_vm<3 * (NB - 1)>();
    } else {
      wait_vm<0>();
    }
    const int s = s0 + u;
    const uint32_t st = stage_base + (uint32_t)slot * kTileBytes;
    slot = slot + 1 == NB ? 0 : slot + 1;
    u32x4 hd = lds_read16(st + b_hd), q0 = lds_read16(st + b_q), q1 = lds_read16<16>(st + b_q);
    lds_wait(hd, q0, q1);
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
      const uint32_t aa = aon ? frag_base + vs * kFragBytes + a_rel : zero_base;
      u32x4 a0 = lds_read16<0>(aa), a1 = lds_read16<16>(aa), a2 = lds_read16<32>(aa), a3 = lds_read16<48>(aa);
      u32x4 mt = lds_read16(meta_base + vs * 64u);
      lds_wait(a0, a1, a2, a3, mt);
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

  // 5. sum over the four groups (lanes j, j+16, j+32, j+48), then over the KQ waves of the tile
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    float sv = acc[v];
    const auto a32 = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(int, sv), __builtin_bit_cast(int, sv), false, false);
    sv = __builtin_bit_cast(float, (int)a32[0]) + __builtin_bit_cast(float, (int)a32[1]);
    const auto a16 = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(int, sv), __builtin_bit_cast(int, sv), false, false);
    acc[v] = __builtin_bit_cast(float, (int)a16[0]) + __builtin_bit_cast(float, (int)a16[1]);
  }
  __syncthreads();  // every wave is done with its stages: reuse the ring for the sums
  float* red = reinterpret_cast<float*>(ring);  // [tq][kq][v][16]
  if (lane < 16) {
#pragma unroll
    for (int v = 0; v < NV; ++v) red[((tq * KQ + kq) * NV + v) * 16 + lane] = acc[v];
  }
  __syncthreads();
  for (int o = tid; o < TQ * NV * 16; o += 1024) {
    const int t = o / (NV * 16), v = (o >> 4) % NV, r = o & 15;
    const int row = 16 * t + r;
    if (row < cnt) {
      float sum = 0.0f;
      for (int k = 0; k < KQ; ++k) sum += red[((t * KQ + k) * NV + v) * 16 + r];
      Y[(size_t)v * rows + rb + row] = sum;
    }
  }
}

constexpr int kCUs = 256;
constexpr size_t kLdsMax = 160 * 1024;

template <int NV, int NB, int TPT>
static void launch_mx(const void* w, const float* X, float* Y, int rows, int cols, const MxGeo& geo, int nwg,
                      hipStream_t s) {
  auto kern = &k_gemv_mx<NV, NB, TPT>;
  const size_t lds = mx_dyn_bytes(NV, geo.nsb);
  (void)hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  kern<<<(unsigned)nwg, 1024u, lds, s>>>(static_cast<const uint8_t*>(w), X, Y, rows, cols, geo);
}

// NB = 3 stages when they fit; TPT = activation conversion tasks per thread.
template <int NV>
static void launch_mx_nv(const void* w, const float* X, float* Y, int rows, int cols, const MxGeo& geo, int nwg,
                         hipStream_t s) {
  const bool nb3 = mx_lds_bytes(NV, geo.nsb, 3) <= kLdsMax;
  const int tpt = (NV * geo.nsb * 32 + 1023) / 1024;
  if (tpt <= 1) return nb3 ? launch_mx<NV, 3, 1>(w, X, Y, rows, cols, geo, nwg, s) : launch_mx<NV, 2, 1>(w, X, Y, rows, cols, geo, nwg, s);
  if (tpt <= 2) return nb3 ? launch_mx<NV, 3, 2>(w, X, Y, rows, cols, geo, nwg, s) : launch_mx<NV, 2, 2>(w, X, Y, rows, cols, geo, nwg, s);
  return nb3 ? launch_mx<NV, 3, 4>(w, X, Y, rows, cols, geo, nwg, s) : launch_mx<NV, 2, 4>(w, X, Y, rows, cols, geo, nwg, s);
}

}  // namespace

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
                        hipStream_t s) {
  const int maxnv = gemv_mx_max_nv(cols);
  if (maxnv == 0 || nvec < 1 || nvec > maxnv || row_bytes >= (1u << 24)) return false;
  MxGeo geo{};
  geo.nsb = cols / 256;
  geo.row_bytes = (uint32_t)row_bytes;
  // one workgroup of 16 waves per CU; tiles of 16 rows; TQ tiles x KQ K-splits per workgroup
  int64_t nwg = std::min<int64_t>(kCUs, ((int64_t)rows + 15) / 16);
  nwg = std::max<int64_t>(nwg, ((int64_t)rows + 255) / 256);
  geo.base = (int)(rows / nwg);
  geo.rem = (int)(rows % nwg);
  const int per = geo.base + (geo.rem ? 1 : 0);
  int tq = 1;
  while (16 * tq < per) tq <<= 1;
  geo.TQ = tq;
  geo.KQ = 16 / tq;
  switch (nvec) {
    case 1: launch_mx_nv<1>(w, X, Y, rows, cols, geo, (int)nwg, s); break;
    case 2: launch_mx_nv<2>(w, X, Y, rows, cols, geo, (int)nwg, s); break;
    case 3: launch_mx_nv<3>(w, X, Y, rows, cols, geo, (int)nwg, s); break;
    case 4: launch_mx_nv<4>(w, X, Y, rows, cols, geo, (int)nwg, s); break;
    case 5: launch_mx_nv<5>(w, X, Y, rows, cols, geo, (int)nwg, s); break;
    case 6: launch_mx_nv<6>(w, X, Y, rows, cols, geo, (int)nwg, s); break;
    case 7: launch_mx_nv<7>(w, X, Y, rows, cols, geo, (int)nwg, s); break;
    default: launch_mx_nv<8>(w, X, Y, rows, cols, geo, (int)nwg, s); break;
  }
  return true;
}

}  // namespace qvx
