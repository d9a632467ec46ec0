// qvx_gemv.hip -- decode GEMV (M = 1..16) over raw GGUF blocks on gfx950.
//
// out[v, r] = sum_k dequant(W)[r, k] * X[v, k]   (the reference's qmatmul / qmatmulN,
// runtime/src/qmatmul.cpp:28-115), fp32 activations, fp32 accumulation.
//
// Work decomposition (one 256-thread workgroup = 4 waves):
//  * A workgroup owns RT = 4*RL consecutive rows and walks K in panels of 2048 elements
//    (PB blocks: 8 super-blocks for Q4_K / Q6_K, 64 blocks for Q4_0 / Q8_0).
//  * Each panel's bytes for the RT rows are streamed with 16-byte global loads (consecutive
//    threads, consecutive 16-byte chunks: fully coalesced), held in registers while the previous
//    panel is computed, then written to an LDS double buffer -- one barrier per panel.
//  * In a panel every lane owns one "slot" of 32 elements at a fixed column position and wave w
//    computes that slot for its RL rows, so each activation value is loaded once per panel and
//    reused across the RL rows (and, for NV <= 2, across rows without reloading).
//  * A slot is two runs of 16 elements (A, B).  Quant fields are unpacked in registers into
//    packed fp16 pairs whose bit patterns are the small integers themselves (fp16 subnormals:
//    q * 2^-24, exact); v_fma_mix_f32 multiplies them straight into fp32 sums with the fp32
//    activations.  The integer sums are rescaled once per run:
//        Q4_K: d*sc*sum(n x) - dmin*m*sum(x)      Q6_K: d*sc*(sum(q x) - 32 sum(x))
//        Q4_0: d*(sum(n x) - 8 sum(x))            Q8_0: d*(sum((q+128) x) - 128 sum(x))
//    which is the dequantised value d*sc*n - dmin*m (etc.) summed in another order; every
//    product is exact, so only fp32 summation error enters (checked at 1e-3 max-relative).
//  * The 64 lane partials of each output are summed by a fixed xor-butterfly.  The per-output
//    arithmetic does not depend on NV, so qvx_qmatmul_n is bit-identical to qvx_qmatmul per
//    vector, the reference's promise for qmatmulN (runtime/include/qorvix/runtime/qmatmul.hpp:31-32).
//
// Requirements checked by the launcher: W 16-byte aligned, row pitch a multiple of 16 bytes,
// X 16-byte aligned.  Other shapes go to the generic kernel in qvx_dequant.hip.
#include "qvx_common.hpp"

namespace qvx {

// ---- LDS byte-stream readers (only 4-byte-aligned ds_read_b32, realigned in registers) --------

__device__ inline uint32_t lds_u32(const uint8_t* lds, int off) {
  return *reinterpret_cast<const uint32_t*>(lds + off);
}

// 16 bytes starting at an arbitrary byte offset.
__device__ inline void lds_read16(const uint8_t* lds, int off, uint32_t (&q)[4]) {
  const int a = off & ~3;
  const uint32_t s = (uint32_t)(off & 3);
  uint32_t e[5];
#pragma unroll
  for (int i = 0; i < 5; ++i) e[i] = lds_u32(lds, a + 4 * i);
#pragma unroll
  for (int i = 0; i < 4; ++i) q[i] = align_bytes(e[i + 1], e[i], s);
}

// 16-bit little-endian field at an even byte offset.
__device__ inline uint32_t lds_u16(const uint8_t* lds, int off) {
  return (lds_u32(lds, off & ~3) >> (8 * (off & 2))) & 0xFFFFu;
}

// Signed byte at any offset.
__device__ inline float lds_i8f(const uint8_t* lds, int off) {
  const uint32_t w = lds_u32(lds, off & ~3);
  return (float)__builtin_amdgcn_sbfe(w, 8 * (off & 3), 8);
}

// ---- a slot: 2 runs x 16 elements as packed fp16 integer pairs + per-run scales --------------
struct Slot {
  uint32_t a[8], b[8];  // pairs: a[2j] = elems (4j, 4j+2), a[2j+1] = elems (4j+1, 4j+3) of run A
  float ka, kb;         // factors turning the raw fp16-subnormal dot of run A / B into sum(q x)
  float ca, cb;         // coefficients of sum(x) over run A / B (offsets and minimums, scaled)
  float d;              // scale of the quant sums
};

// Splits 4 bytes of 4-bit fields (low nibbles) into two packed-half dwords, as fp16 subnormals.
__device__ inline void nib_lo(uint32_t w, uint32_t& p02, uint32_t& p13) {
  p02 = w & 0x000F000Fu;
  p13 = (w >> 8) & 0x000F000Fu;
}
// High nibbles, left in place (value 16*n as fp16 subnormal): the caller scales by 2^20.
__device__ inline void nib_hi(uint32_t w, uint32_t& p02, uint32_t& p13) {
  p02 = w & 0x00F000F0u;
  p13 = (w >> 8) & 0x00F000F0u;
}

constexpr float k2p24 = 16777216.0f;  // 2^24
constexpr float k2p20 = 1048576.0f;   // 2^20

template <uint32_t T> struct SlotOps;

// Q4_K: slot s of a panel = super-block b = s/8, 16-byte quant chunk k = s%8 of its 128 qs bytes.
// Chunk k holds bytes l = 16(k%2)..+15 of 64-element group c = k/2: low nibbles are sub-block 2c
// (elements 64c + l), high nibbles sub-block 2c+1 (elements 64c + 32 + l).
template <> struct SlotOps<T_Q4_K> {
  static __device__ inline int xa(int s) { return 256 * (s >> 3) + 64 * ((s & 7) >> 1) + 16 * (s & 1); }
  static constexpr int kXB = 32;  // run B = run A + 32 elements
  static __device__ inline int block(int s) { return s >> 3; }
  static __device__ inline void decode(const uint8_t* lrow, int s, Slot& o) {
    const int b = s >> 3, k = s & 7, c = k >> 1;
    const uint4 h = *reinterpret_cast<const uint4*>(lrow + 144 * b);
    const uint4 q = *reinterpret_cast<const uint4*>(lrow + 144 * b + 16 + 16 * k);
    const uint32_t qq[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      nib_lo(qq[j], o.a[2 * j], o.a[2 * j + 1]);
      nib_hi(qq[j], o.b[2 * j], o.b[2 * j + 1]);
    }
    // 6-bit (scale, min) of sub-blocks 2c and 2c+1 as byte pairs (public K-quant scale packing).
    uint32_t scp, mp;
    if (c < 2) {
      const uint32_t sh = 16u * (uint32_t)c;
      scp = (h.y >> sh) & 0x3F3Fu;
      mp = (h.z >> sh) & 0x3F3Fu;
    } else {
      const uint32_t sh = 16u * (uint32_t)(c - 2);
      scp = ((h.w >> sh) & 0x0F0Fu) | ((h.y >> (sh + 2)) & 0x3030u);
      mp = ((h.w >> (sh + 4)) & 0x0F0Fu) | ((h.z >> (sh + 2)) & 0x3030u);
    }
    o.ka = (float)(scp & 0xFFu) * k2p24;
    o.kb = (float)(scp >> 8) * k2p20;
    const float dmin = f16hi(h.x);
    o.d = f16lo(h.x);
    // sum = d*(ka*dotA + kb*dotB) - dmin*(ma*sxA + mb*sxB); dmin*m is exact in fp32.
    o.ca = -dmin * (float)(mp & 0xFFu);
    o.cb = -dmin * (float)(mp >> 8);
  }
};

// Q6_K: slot s = super-block b = s/8, u = s%8 -> half h = u/4, l-group t = (u/2)%2, e = u%2.
// It covers quarters e (low nibbles of ql[64h + 32e + 16t ..+16]) and e+2 (their high nibbles),
// with 2-bit high parts from qh[32h + 16t ..+16] bits (2e, 2e+1) and (2e+4, 2e+5).
template <> struct SlotOps<T_Q6_K> {
  static __device__ inline int xa(int s) {
    const int u = s & 7;
    return 256 * (s >> 3) + 128 * (u >> 2) + 32 * (u & 1) + 16 * ((u >> 1) & 1);
  }
  static constexpr int kXB = 64;
  static __device__ inline int block(int s) { return s >> 3; }
  static __device__ inline void decode(const uint8_t* lrow, int s, Slot& o) {
    const int b = s >> 3, u = s & 7, h = u >> 2, t = (u >> 1) & 1, e = u & 1;
    const int base = 210 * b;
    uint32_t ql[4], qh[4];
    lds_read16(lrow, base + 64 * h + 32 * e + 16 * t, ql);
    lds_read16(lrow, base + 128 + 32 * h + 16 * t, qh);
    const uint32_t shl = 4u - 2u * (uint32_t)e, shr = 2u * (uint32_t)e;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t ha = qh[j] << shl;  // bits (2e, 2e+1) of each byte -> bits 4..5
      const uint32_t hb = qh[j] >> shr;  // bits (2e+4, 2e+5) of each byte -> bits 4..5
      o.a[2 * j] = (ql[j] & 0x000F000Fu) | (ha & 0x00300030u);
      o.a[2 * j + 1] = ((ql[j] >> 8) & 0x000F000Fu) | ((ha >> 8) & 0x00300030u);
      o.b[2 * j] = ((ql[j] >> 4) & 0x000F000Fu) | (hb & 0x00300030u);
      o.b[2 * j + 1] = ((ql[j] >> 12) & 0x000F000Fu) | ((hb >> 8) & 0x00300030u);
    }
    const float sa = lds_i8f(lrow, base + 192 + 8 * h + t + 2 * e);
    const float sb = lds_i8f(lrow, base + 192 + 8 * h + t + 2 * e + 4);
    o.d = f16lo(lds_u16(lrow, base + 208));
    o.ka = sa * k2p24;
    o.kb = sb * k2p24;
    o.ca = -32.0f * (o.d * sa);  // d * int8 scale * 32: exact
    o.cb = -32.0f * (o.d * sb);
  }
};

// Q4_0: slot s = block s; low nibbles of qs[i] are element i (run A), high nibbles element 16+i.
template <> struct SlotOps<T_Q4_0> {
  static __device__ inline int xa(int s) { return 32 * s; }
  static constexpr int kXB = 16;
  static __device__ inline int block(int s) { return s; }
  static __device__ inline void decode(const uint8_t* lrow, int s, Slot& o) {
    const int base = 18 * s;
    uint32_t q[4];
    lds_read16(lrow, base + 2, q);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      nib_lo(q[j], o.a[2 * j], o.a[2 * j + 1]);
      nib_hi(q[j], o.b[2 * j], o.b[2 * j + 1]);
    }
    o.d = f16lo(lds_u16(lrow, base));
    o.ka = k2p24;
    o.kb = k2p20;
    o.ca = -8.0f * o.d;
    o.cb = o.ca;
  }
};

// Q8_0: slot s = block s; int8 quants biased to q+128 (one xor) so they are unsigned fp16
// subnormals; run A = elements 0..15, run B = 16..31.
template <> struct SlotOps<T_Q8_0> {
  static __device__ inline int xa(int s) { return 32 * s; }
  static constexpr int kXB = 16;
  static __device__ inline int block(int s) { return s; }
  static __device__ inline void decode(const uint8_t* lrow, int s, Slot& o) {
    const int base = 34 * s;
    uint32_t q0[4], q1[4];
    lds_read16(lrow, base + 2, q0);
    lds_read16(lrow, base + 18, q1);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t u0 = q0[j] ^ 0x80808080u, u1 = q1[j] ^ 0x80808080u;
      o.a[2 * j] = u0 & 0x00FF00FFu;
      o.a[2 * j + 1] = (u0 >> 8) & 0x00FF00FFu;
      o.b[2 * j] = u1 & 0x00FF00FFu;
      o.b[2 * j + 1] = (u1 >> 8) & 0x00FF00FFu;
    }
    o.d = f16lo(lds_u16(lrow, base));
    o.ka = k2p24;
    o.kb = k2p24;
    o.ca = -128.0f * o.d;
    o.cb = o.ca;
  }
};

// Sum over 16 elements of (packed fp16 integer) * x in element order, fp32 fused steps.
__device__ inline float dot16(const uint32_t (&p)[8], const float (&x)[16]) {
  float acc = 0.0f;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    acc = __builtin_fmaf(f16lo(p[2 * j]), x[4 * j + 0], acc);
    acc = __builtin_fmaf(f16lo(p[2 * j + 1]), x[4 * j + 1], acc);
    acc = __builtin_fmaf(f16hi(p[2 * j]), x[4 * j + 2], acc);
    acc = __builtin_fmaf(f16hi(p[2 * j + 1]), x[4 * j + 3], acc);
  }
  return acc;
}

__device__ inline float sum16(const float (&x)[16]) {
  float s = 0.0f;
#pragma unroll
  for (int i = 0; i < 16; ++i) s += x[i];
  return s;
}

__device__ inline void load16(const float* p, float (&x)[16]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float4 v = reinterpret_cast<const float4*>(p)[i];
    x[4 * i] = v.x;
    x[4 * i + 1] = v.y;
    x[4 * i + 2] = v.z;
    x[4 * i + 3] = v.w;
  }
}

// acc + d*(ka*dotA + kb*dotB) + (ca*sxA + cb*sxB), in a fixed sequence of fused steps.
__device__ inline float combine(const Slot& o, float dA, float dB, float sxA, float sxB, float acc) {
  float t = o.ka * dA;
  t = __builtin_fmaf(o.kb, dB, t);
  float u = o.ca * sxA;
  u = __builtin_fmaf(o.cb, sxB, u);
  return __builtin_fmaf(o.d, t, acc) + u;
}

__device__ inline float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

template <uint32_t T, int NV, int RL>
__global__ __launch_bounds__(256) void k_gemv(const uint8_t* __restrict__ W, const float* __restrict__ X,
                                              float* __restrict__ Y, int rows, int cols, int nblk,
                                              size_t row_bytes) {
  using F = Fmt<T>;
  using S = SlotOps<T>;
  constexpr int RT = 4 * RL;                 // rows per workgroup
  constexpr int PBY = F::PB * F::BB;         // panel bytes per row (multiple of 16)
  constexpr int NCH = PBY / 16;              // 16-byte chunks per row panel
  constexpr int LSTR = PBY + 16;             // LDS row pitch: +16 so aligned over-reads stay inside
  constexpr int NLD = (RT * NCH + 255) / 256;
  __shared__ __attribute__((aligned(16))) uint8_t lds[2][RT * LSTR];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int row0 = blockIdx.x * RT;
  const int npan = (nblk + F::PB - 1) / F::PB;

  uint4 st[NLD];
  auto gload = [&](int p) {
    const int nbp = min(F::PB, nblk - p * F::PB);
    const int nch = (nbp * F::BB + 15) >> 4;
#pragma unroll
    for (int j = 0; j < NLD; ++j) {
      const int q = tid + 256 * j;
      const int r = q / NCH, c = q - r * NCH;
      if (q < RT * NCH && c < nch && row0 + r < rows)
        st[j] = *reinterpret_cast<const uint4*>(W + (size_t)(row0 + r) * row_bytes + (size_t)p * PBY + 16 * c);
    }
  };
  auto lstore = [&](int buf) {
#pragma unroll
    for (int j = 0; j < NLD; ++j) {
      const int q = tid + 256 * j;
      const int r = q / NCH, c = q - r * NCH;
      if (q < RT * NCH) *reinterpret_cast<uint4*>(&lds[buf][r * LSTR + 16 * c]) = st[j];
    }
  };

  float acc[RL][NV];
#pragma unroll
  for (int i = 0; i < RL; ++i)
#pragma unroll
    for (int v = 0; v < NV; ++v) acc[i][v] = 0.0f;

  gload(0);
  for (int p = 0; p < npan; ++p) {
    const int buf = p & 1;
    lstore(buf);
    __syncthreads();
    if (p + 1 < npan) gload(p + 1);

    const int nbp = min(F::PB, nblk - p * F::PB);
    if (S::block(lane) < nbp) {
      const float* xp = X + (size_t)p * 2048 + S::xa(lane);
      if constexpr (NV <= 2) {
        float xa[NV][16], xb[NV][16], sa[NV], sb[NV];
#pragma unroll
        for (int v = 0; v < NV; ++v) {
          load16(xp + (size_t)v * cols, xa[v]);
          load16(xp + (size_t)v * cols + S::kXB, xb[v]);
          sa[v] = sum16(xa[v]);
          sb[v] = sum16(xb[v]);
        }
#pragma unroll
        for (int i = 0; i < RL; ++i) {
          const int r = wave * RL + i;
          if (row0 + r < rows) {
            Slot o;
            S::decode(&lds[buf][r * LSTR], lane, o);
#pragma unroll
            for (int v = 0; v < NV; ++v)
              acc[i][v] = combine(o, dot16(o.a, xa[v]), dot16(o.b, xb[v]), sa[v], sb[v], acc[i][v]);
          }
        }
      } else {
        float sa[NV], sb[NV];
#pragma unroll
        for (int v = 0; v < NV; ++v) {
          float xa[16], xb[16];
          load16(xp + (size_t)v * cols, xa);
          load16(xp + (size_t)v * cols + S::kXB, xb);
          sa[v] = sum16(xa);
          sb[v] = sum16(xb);
        }
#pragma unroll
        for (int i = 0; i < RL; ++i) {
          const int r = wave * RL + i;
          if (row0 + r < rows) {
            Slot o;
            S::decode(&lds[buf][r * LSTR], lane, o);
#pragma unroll
            for (int v = 0; v < NV; ++v) {
              float xa[16], xb[16];
              load16(xp + (size_t)v * cols, xa);
              load16(xp + (size_t)v * cols + S::kXB, xb);
              acc[i][v] = combine(o, dot16(o.a, xa), dot16(o.b, xb), sa[v], sb[v], acc[i][v]);
            }
          }
        }
      }
    }
  }

#pragma unroll
  for (int i = 0; i < RL; ++i) {
    const int r = row0 + wave * RL + i;
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      const float s = wave_sum(acc[i][v]);
      if (lane == 0 && r < rows) Y[(size_t)v * rows + r] = s;
    }
  }
}

// ---- launch ---------------------------------------------------------------------------------

template <uint32_t T, int NV, int RL>
static void launch_t(const void* w, const float* X, float* Y, int rows, int cols, size_t row_bytes, hipStream_t s) {
  constexpr int RT = 4 * RL;
  const int nblk = cols / Fmt<T>::QK;
  const unsigned grid = (unsigned)((rows + RT - 1) / RT);
  k_gemv<T, NV, RL><<<grid, 256, 0, s>>>(static_cast<const uint8_t*>(w), X, Y, rows, cols, nblk, row_bytes);
}

// Rows per lane: enough workgroups to cover 256 CUs several times, LDS within budget.
template <uint32_t T, int NV>
static void launch_nv(const void* w, const float* X, float* Y, int rows, int cols, size_t row_bytes,
                      hipStream_t s) {
  if constexpr (NV <= 2) {
    if (rows >= 16384) return launch_t<T, NV, 4>(w, X, Y, rows, cols, row_bytes, s);
    if (rows >= 4096) return launch_t<T, NV, 2>(w, X, Y, rows, cols, row_bytes, s);
    return launch_t<T, NV, 1>(w, X, Y, rows, cols, row_bytes, s);
  } else {
    if (rows >= 8192) return launch_t<T, NV, 2>(w, X, Y, rows, cols, row_bytes, s);
    return launch_t<T, NV, 1>(w, X, Y, rows, cols, row_bytes, s);
  }
}

template <uint32_t T>
static void launch_type(const void* w, const float* X, float* Y, int nvec, int rows, int cols,
                        size_t row_bytes, hipStream_t s) {
  switch (nvec) {
    case 1: return launch_nv<T, 1>(w, X, Y, rows, cols, row_bytes, s);
    case 2: return launch_nv<T, 2>(w, X, Y, rows, cols, row_bytes, s);
    case 3: return launch_nv<T, 3>(w, X, Y, rows, cols, row_bytes, s);
    case 4: return launch_nv<T, 4>(w, X, Y, rows, cols, row_bytes, s);
    case 5: return launch_nv<T, 5>(w, X, Y, rows, cols, row_bytes, s);
    case 6: return launch_nv<T, 6>(w, X, Y, rows, cols, row_bytes, s);
    case 7: return launch_nv<T, 7>(w, X, Y, rows, cols, row_bytes, s);
    case 8: return launch_nv<T, 8>(w, X, Y, rows, cols, row_bytes, s);
    case 9: return launch_nv<T, 9>(w, X, Y, rows, cols, row_bytes, s);
    case 10: return launch_nv<T, 10>(w, X, Y, rows, cols, row_bytes, s);
    case 11: return launch_nv<T, 11>(w, X, Y, rows, cols, row_bytes, s);
    case 12: return launch_nv<T, 12>(w, X, Y, rows, cols, row_bytes, s);
    case 13: return launch_nv<T, 13>(w, X, Y, rows, cols, row_bytes, s);
    case 14: return launch_nv<T, 14>(w, X, Y, rows, cols, row_bytes, s);
    case 15: return launch_nv<T, 15>(w, X, Y, rows, cols, row_bytes, s);
    default: return launch_nv<T, 16>(w, X, Y, rows, cols, row_bytes, s);
  }
}

// Fast-path GEMV for 1 <= nvec <= 16 on 16-byte-aligned rows of Q8_0 / Q4_0 / Q4_K / Q6_K.
bool launch_gemv_fast(uint32_t t, const void* w, const float* X, float* Y, int nvec, int rows, int cols,
                      size_t row_bytes, hipStream_t s) {
  switch (t) {
    case T_Q4_K: launch_type<T_Q4_K>(w, X, Y, nvec, rows, cols, row_bytes, s); return true;
    case T_Q6_K: launch_type<T_Q6_K>(w, X, Y, nvec, rows, cols, row_bytes, s); return true;
    case T_Q4_0: launch_type<T_Q4_0>(w, X, Y, nvec, rows, cols, row_bytes, s); return true;
    case T_Q8_0: launch_type<T_Q8_0>(w, X, Y, nvec, rows, cols, row_bytes, s); return true;
    default: return false;
  }
}

}  // namespace qvx
