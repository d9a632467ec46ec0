// qvx_gemv.hip -- decode GEMV (M = 1..16) over raw GGUF blocks on gfx950.
//
// out[v, r] = sum_k dequant(W)[r, k] * X[v, k]   (the reference's qmatmul / qmatmulN,
// runtime/src/qmatmul.cpp:28-115), fp32 activations, fp32 accumulation.
//
// Work decomposition:
//  * A row of K = cols elements is cut into S = K/32 "slots" of 32 elements (one Q4_0 / Q8_0
//    block, or one eighth of a Q4_K / Q6_K super-block).  A workgroup has G groups of S' lanes
//    (S' = S rounded up to a multiple of 64, or to a power of two when S < 64); lane j of a group
//    owns slot j for the whole kernel, so its activation values (32 floats per vector) and their
//    run sums are loaded and formed once and reused for every row it touches.
//  * Each lane walks RL rows (group g takes rows g, g+G, ... of the workgroup's G*RL rows).  All
//    RL rows' quant bytes are requested up front with direct global loads into registers
//    (16-byte loads where the block layout is 16-byte aligned -- Q4_K -- and dword-aligned
//    dwordx4 + tail loads realigned with v_alignbyte where it is not), then consumed in issue
//    order, so each row is computed as soon as its bytes land while later rows are in flight.
//  * Quant fields are unpacked in registers into packed fp16 pairs whose bit patterns are the
//    small integers themselves (fp16 subnormals q * 2^-24, exact); v_fma_mix_f32 multiplies them
//    straight into fp32 sums with the fp32 activations.  Per run of 16 the integer sums are
//    rescaled once:  Q4_K: d*sc*sum(n x) - dmin*m*sum(x);  Q6_K: d*sc*(sum(q x) - 32 sum(x));
//    Q4_0: d*(sum(n x) - 8 sum(x));  Q8_0: d*(sum((q+128) x) - 128 sum(x)).  Every product is
//    exact, so only fp32 summation error enters (checked at 1e-3 max-relative).
//  * Each output's S' lane partials are summed by a fixed xor butterfly inside each wave and, for
//    groups wider than a wave, by one thread over the wave sums in wave order.  None of this
//    depends on NV, so qvx_qmatmul_n is bit-identical to qvx_qmatmul per vector, the reference's
//    promise for qmatmulN (runtime/include/qorvix/runtime/qmatmul.hpp:31-32).
//
// Requirements checked by the launcher: W and X 16-byte aligned, row pitch a multiple of 16 bytes,
// S' <= 1024.  Other shapes go to the generic kernel in qvx_dequant.hip.
#include "qvx_common.hpp"

namespace qvx {

typedef uint32_t u32x4a4_t __attribute__((ext_vector_type(4), aligned(4)));  // dword-aligned 16 bytes

__device__ inline uint4 ldg16(const uint8_t* p) {  // p 16-byte aligned
  return *reinterpret_cast<const uint4*>(p);
}
__device__ inline u32x4a4_t ldg16a4(const uint8_t* p) {  // p 4-byte aligned
  return *reinterpret_cast<const u32x4a4_t*>(p);
}
__device__ inline uint32_t ldg4(const uint8_t* p) { return *reinterpret_cast<const uint32_t*>(p); }
__device__ inline uint32_t ldg2(const uint8_t* p) { return *reinterpret_cast<const uint16_t*>(p); }

// 16 bytes starting at byte offset s (0..3) of the 20-byte window (w, e).
__device__ inline void realign16(const u32x4a4_t& w, uint32_t e, uint32_t s, uint32_t (&q)[4]) {
  q[0] = align_bytes(w.y, w.x, s);
  q[1] = align_bytes(w.z, w.y, s);
  q[2] = align_bytes(w.w, w.z, s);
  q[3] = align_bytes(e, w.w, s);
}

// ---- a slot: 2 runs x 16 elements as packed fp16 integer pairs + per-run scales --------------
struct Slot {
  uint32_t a[8], b[8];  // pairs: a[2j] = elems (4j, 4j+2), a[2j+1] = elems (4j+1, 4j+3) of run A
  float ka, kb;         // factors turning the raw fp16-subnormal dot of run A / B into sum(q x)
  float ca, cb;         // coefficients of sum(x) over run A / B (offsets and minimums, scaled)
  float d;              // scale of the quant sums
};

// Low nibbles of 4 bytes as two packed-half dwords (fp16 subnormals n * 2^-24).
__device__ inline void nib_lo(uint32_t w, uint32_t& p02, uint32_t& p13) {
  p02 = w & 0x000F000Fu;
  p13 = (w >> 8) & 0x000F000Fu;
}
// High nibbles left in place (16 * n as fp16 subnormal): the caller scales by 2^20.
__device__ inline void nib_hi(uint32_t w, uint32_t& p02, uint32_t& p13) {
  p02 = w & 0x00F000F0u;
  p13 = (w >> 8) & 0x00F000F0u;
}

constexpr float k2p24 = 16777216.0f;  // 2^24
constexpr float k2p20 = 1048576.0f;   // 2^20

// Per-type lane logic: Raw = the registers one row's slot needs; load() issues the global loads
// (rows are 16-byte aligned; offsets below are row-relative); unpack() turns Raw into a Slot;
// xoff() is the slot's run-A offset within the row (run B = run A + kXB).
template <uint32_t T> struct Lane;

// Q4_K: slot = super-block b = sig/8, 16-byte quant chunk k = sig%8 of its 128 qs bytes.  Chunk k
// holds bytes l = 16(k%2)..+15 of 64-element group c = k/2: low nibbles are sub-block 2c
// (elements 64c + l), high nibbles sub-block 2c+1 (elements 64c + 32 + l).
template <> struct Lane<T_Q4_K> {
  static constexpr int kSPB = 8, kXB = 32;
  struct Raw {
    uint4 q, h;
  };
  static __device__ inline int xoff(int sig) { return 256 * (sig >> 3) + 64 * ((sig & 7) >> 1) + 16 * (sig & 1); }
  static __device__ inline void load(const uint8_t* row, int sig, Raw& r) {
    const uint8_t* blk = row + 144 * (sig >> 3);
    r.h = ldg16(blk);
    r.q = ldg16(blk + 16 + 16 * (sig & 7));
  }
  static __device__ inline void unpack(const Raw& r, int sig, Slot& o) {
    const uint32_t qq[4] = {r.q.x, r.q.y, r.q.z, r.q.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      nib_lo(qq[j], o.a[2 * j], o.a[2 * j + 1]);
      nib_hi(qq[j], o.b[2 * j], o.b[2 * j + 1]);
    }
    // 6-bit (scale, min) of sub-blocks 2c, 2c+1 as byte pairs (public K-quant scale packing):
    // c < 2: sc = s[2c..] & 63, m = s[2c+4..] & 63; c >= 2: low 4 bits from s[2c+4..], high 2 bits
    // from bits 6-7 of s[2c-4..] (scale) and s[2c..] (min).  Branch-free: c is lane-constant.
    const int c = (sig & 7) >> 1;
    const bool hi = c >= 2;
    const uint32_t sh = 16u * (uint32_t)(c & 1);
    const uint32_t m1 = hi ? 0x0F0Fu : 0x3F3Fu, m2 = hi ? 0x3030u : 0u;
    const uint32_t scp = (((hi ? r.h.w : r.h.y) >> sh) & m1) | ((r.h.y >> (sh + 2)) & m2);
    const uint32_t mp = (((hi ? r.h.w : r.h.z) >> (sh + (hi ? 4u : 0u))) & m1) | ((r.h.z >> (sh + 2)) & m2);
    o.ka = (float)(scp & 0xFFu) * k2p24;
    o.kb = (float)(scp >> 8) * k2p20;
    const float dmin = f16hi(r.h.x);
    o.d = f16lo(r.h.x);
    o.ca = -dmin * (float)(mp & 0xFFu);  // dmin * m is exact in fp32
    o.cb = -dmin * (float)(mp >> 8);
  }
};

// Q6_K: slot = super-block b = sig/8, u = sig%8 -> half h = u/4, l-group t = (u/2)%2, e = u%2.
// It covers quarter e (low nibbles of ql[64h + 32e + 16t ..+16]) and quarter e+2 (their high
// nibbles) with 2-bit high parts from qh[32h + 16t ..+16], bits (2e, 2e+1) and (2e+4, 2e+5);
// scales sc[8h + t + 2e] and sc[8h + t + 2e + 4].  Super-blocks are 2-byte aligned: each 16-byte
// piece is read as a dword-aligned 20-byte window (never past its super-block) and realigned.
template <> struct Lane<T_Q6_K> {
  static constexpr int kSPB = 8, kXB = 64;
  struct Raw {
    u32x4a4_t l, h;
    uint32_t le, he, s0, s1, dd;
    uint32_t sh;  // byte misalignment of the pieces (0 or 2)
    uint32_t ssh; // byte position of the first scale inside s0
  };
  static __device__ inline int xoff(int sig) {
    const int u = sig & 7;
    return 256 * (sig >> 3) + 128 * (u >> 2) + 32 * (u & 1) + 16 * ((u >> 1) & 1);
  }
  static __device__ inline void load(const uint8_t* row, int sig, Raw& r) {
    const int b = sig >> 3, u = sig & 7, h = u >> 2, t = (u >> 1) & 1, e = u & 1;
    const int base = 210 * b;
    const int ol = base + 64 * h + 32 * e + 16 * t, oh = base + 128 + 32 * h + 16 * t;
    const int os = base + 192 + 8 * h + t + 2 * e;
    r.sh = (uint32_t)(ol & 3);
    r.l = ldg16a4(row + (ol & ~3));
    r.le = ldg4(row + (ol & ~3) + 16);
    r.h = ldg16a4(row + (oh & ~3));
    r.he = ldg4(row + (oh & ~3) + 16);
    r.ssh = (uint32_t)(os & 3);
    r.s0 = ldg4(row + (os & ~3));
    r.s1 = ldg4(row + (os & ~3) + 4);
    r.dd = ldg2(row + base + 208);
  }
  static __device__ inline void unpack(const Raw& r, int sig, Slot& o) {
    const uint32_t e = (uint32_t)(sig & 1);
    uint32_t ql[4], qh[4];
    realign16(r.l, r.le, r.sh, ql);
    realign16(r.h, r.he, r.sh, qh);
    const uint32_t shl = 4u - 2u * e, shr = 2u * e;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t ha = qh[j] << shl;  // bits (2e, 2e+1) of each byte -> bits 4..5
      const uint32_t hb = qh[j] >> shr;  // bits (2e+4, 2e+5) of each byte -> bits 4..5
      o.a[2 * j] = (ql[j] & 0x000F000Fu) | (ha & 0x00300030u);
      o.a[2 * j + 1] = ((ql[j] >> 8) & 0x000F000Fu) | ((ha >> 8) & 0x00300030u);
      o.b[2 * j] = ((ql[j] >> 4) & 0x000F000Fu) | (hb & 0x00300030u);
      o.b[2 * j + 1] = ((ql[j] >> 12) & 0x000F000Fu) | ((hb >> 8) & 0x00300030u);
    }
    // sc[.. + 4] is 4 bytes later: same byte position in the next dword.
    const float sa = (float)(int)__builtin_amdgcn_sbfe((int)r.s0, 8u * r.ssh, 8u);
    const float sb = (float)(int)__builtin_amdgcn_sbfe((int)r.s1, 8u * r.ssh, 8u);
    o.d = f16lo(r.dd);
    o.ka = sa * k2p24;
    o.kb = sb * k2p24;
    o.ca = -32.0f * (o.d * sa);  // d * int8 scale * 32: exact
    o.cb = -32.0f * (o.d * sb);
  }
};

// Q4_0: slot = block sig; low nibbles of qs[i] are element i (run A), high nibbles element 16+i.
template <> struct Lane<T_Q4_0> {
  static constexpr int kSPB = 1, kXB = 16;
  struct Raw {
    u32x4a4_t q;
    uint32_t qe, dd, sh;
  };
  static __device__ inline int xoff(int sig) { return 32 * sig; }
  static __device__ inline void load(const uint8_t* row, int sig, Raw& r) {
    const int base = 18 * sig, o = base + 2;
    r.sh = (uint32_t)(o & 3);
    r.q = ldg16a4(row + (o & ~3));
    r.qe = ldg2(row + (o & ~3) + 16);  // 2 bytes: the window never passes the block's end
    r.dd = ldg2(row + base);
  }
  static __device__ inline void unpack(const Raw& r, int, Slot& o) {
    uint32_t q[4];
    realign16(r.q, r.qe, r.sh, q);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      nib_lo(q[j], o.a[2 * j], o.a[2 * j + 1]);
      nib_hi(q[j], o.b[2 * j], o.b[2 * j + 1]);
    }
    o.d = f16lo(r.dd);
    o.ka = k2p24;
    o.kb = k2p20;
    o.ca = -8.0f * o.d;
    o.cb = o.ca;
  }
};

// Q8_0: slot = block sig; int8 quants biased to q+128 (one xor) so they are unsigned fp16
// subnormals; run A = elements 0..15, run B = 16..31.
template <> struct Lane<T_Q8_0> {
  static constexpr int kSPB = 1, kXB = 16;
  struct Raw {
    u32x4a4_t q0, q1;
    uint32_t qe, dd, sh;
  };
  static __device__ inline int xoff(int sig) { return 32 * sig; }
  static __device__ inline void load(const uint8_t* row, int sig, Raw& r) {
    const int base = 34 * sig, o = base + 2;
    const uint8_t* a = row + (o & ~3);
    r.sh = (uint32_t)(o & 3);
    r.q0 = ldg16a4(a);
    r.q1 = ldg16a4(a + 16);
    r.qe = ldg2(a + 32);  // 2 bytes: the window never passes the block's end
    r.dd = ldg2(row + base);
  }
  static __device__ inline void unpack(const Raw& r, int, Slot& o) {
    uint32_t q0[4], q1[4];
    realign16(r.q0, r.q1.x, r.sh, q0);
    realign16(r.q1, r.qe, r.sh, q1);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t u0 = q0[j] ^ 0x80808080u, u1 = q1[j] ^ 0x80808080u;
      o.a[2 * j] = u0 & 0x00FF00FFu;
      o.a[2 * j + 1] = (u0 >> 8) & 0x00FF00FFu;
      o.b[2 * j] = u1 & 0x00FF00FFu;
      o.b[2 * j + 1] = (u1 >> 8) & 0x00FF00FFu;
    }
    o.d = f16lo(r.dd);
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

// Fixed xor butterfly over the low `width` lanes' partner set (width = 64 or a power of two < 64).
__device__ inline float group_sum(float v, int width) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1)
    if (off < width) v += __shfl_xor(v, off, 64);
  return v;
}

template <uint32_t T, int NV, int RL>
__global__ __launch_bounds__(1024) void k_gemv(const uint8_t* __restrict__ W, const float* __restrict__ X,
                                               float* __restrict__ Y, int rows, int cols, size_t row_bytes,
                                               int S, int Sp, int G) {
  using L = Lane<T>;
  __shared__ float red[16][16];  // [output of the group][wave of the group] for groups wider than a wave
  const int tid = threadIdx.x;
  const int g = tid / Sp, sig = tid - g * Sp;
  const int row0 = blockIdx.x * G * RL;
  const bool active = sig < S;
  float acc[RL][NV];
#pragma unroll
  for (int i = 0; i < RL; ++i)
#pragma unroll
    for (int v = 0; v < NV; ++v) acc[i][v] = 0.0f;

  if (active) {
    // this lane's rows: row0 + g + G*i; issue every row's loads before using any of them
    typename L::Raw raw[RL];
#pragma unroll
    for (int i = 0; i < RL; ++i) {
      const int r = min(row0 + g + G * i, rows - 1);  // clamp: past-the-end rows recompute a valid row
      L::load(W + (size_t)r * row_bytes, sig, raw[i]);
    }
    const float* xp = X + L::xoff(sig);
    if constexpr (NV <= 2) {
      float xa[NV][16], xb[NV][16], sa[NV], sb[NV];
#pragma unroll
      for (int v = 0; v < NV; ++v) {
        load16(xp + (size_t)v * cols, xa[v]);
        load16(xp + (size_t)v * cols + L::kXB, xb[v]);
        sa[v] = sum16(xa[v]);
        sb[v] = sum16(xb[v]);
      }
#pragma unroll
      for (int i = 0; i < RL; ++i) {
        Slot o;
        L::unpack(raw[i], sig, o);
#pragma unroll
        for (int v = 0; v < NV; ++v)
          acc[i][v] = combine(o, dot16(o.a, xa[v]), dot16(o.b, xb[v]), sa[v], sb[v], acc[i][v]);
      }
    } else {
      float sa[NV], sb[NV];
#pragma unroll
      for (int v = 0; v < NV; ++v) {
        float xa[16], xb[16];
        load16(xp + (size_t)v * cols, xa);
        load16(xp + (size_t)v * cols + L::kXB, xb);
        sa[v] = sum16(xa);
        sb[v] = sum16(xb);
      }
#pragma unroll
      for (int i = 0; i < RL; ++i) {
        Slot o;
        L::unpack(raw[i], sig, o);
#pragma unroll
        for (int v = 0; v < NV; ++v) {
          float xa[16], xb[16];
          load16(xp + (size_t)v * cols, xa);
          load16(xp + (size_t)v * cols + L::kXB, xb);
          acc[i][v] = combine(o, dot16(o.a, xa), dot16(o.b, xb), sa[v], sb[v], acc[i][v]);
        }
      }
    }
  }

  // ---- reduction over the group's S' lanes (fixed order) -----------------------------------
  const int lane = tid & 63;
  if (Sp <= 64) {
#pragma unroll
    for (int i = 0; i < RL; ++i) {
      const int r = row0 + g + G * i;
#pragma unroll
      for (int v = 0; v < NV; ++v) {
        const float s = group_sum(acc[i][v], Sp);
        if (sig == 0 && r < rows) Y[(size_t)v * rows + r] = s;
      }
    }
  } else {
    const int wig = sig >> 6, nw = Sp >> 6;  // wave index within the group, waves per group
    // outputs in chunks of 16 so the LDS table stays small for any RL * NV
    constexpr int NO = RL * NV;
#pragma unroll
    for (int o0 = 0; o0 < NO; o0 += 16) {
#pragma unroll
      for (int o = o0; o < NO && o < o0 + 16; ++o) {
        const float s = group_sum(acc[o / NV][o % NV], 64);
        if (lane == 0) red[o - o0][g * nw + wig] = s;
      }
      __syncthreads();
      // one thread per (group, output): sum the group's wave partials in wave order
      const int gg = tid / 16, oo = tid % 16;
      if (gg < G && o0 + oo < NO) {
        float s = 0.0f;
        for (int w = 0; w < nw; ++w) s += red[oo][gg * nw + w];
        const int i = (o0 + oo) / NV, v = (o0 + oo) % NV;
        const int r = row0 + gg + G * i;
        if (r < rows) Y[(size_t)v * rows + r] = s;
      }
      __syncthreads();
    }
  }
}

// ---- launch ---------------------------------------------------------------------------------

template <uint32_t T, int NV, int RL>
static void launch_t(const void* w, const float* X, float* Y, int rows, int cols, size_t row_bytes, int S, int Sp,
                     int G, hipStream_t s) {
  const int rt = G * RL;
  const unsigned grid = (unsigned)((rows + rt - 1) / rt);
  k_gemv<T, NV, RL><<<grid, G * Sp, 0, s>>>(static_cast<const uint8_t*>(w), X, Y, rows, cols, row_bytes, S, Sp, G);
}

// Rows per lane: enough rows in flight per lane to cover HBM latency, few enough to keep
// 2-4 waves per SIMD resident and >= ~2 workgroups per CU.
template <uint32_t T, int NV>
static void launch_nv(const void* w, const float* X, float* Y, int rows, int cols, size_t row_bytes, int S, int Sp,
                      int G, hipStream_t s) {
  constexpr bool big = T == T_Q4_K || T == T_Q4_0;  // fewer raw registers per row
  if constexpr (NV == 1) {
    if (rows >= 256 * 8 * G) return launch_t<T, NV, big ? 8 : 4>(w, X, Y, rows, cols, row_bytes, S, Sp, G, s);
    if (rows >= 256 * 4 * G) return launch_t<T, NV, 4>(w, X, Y, rows, cols, row_bytes, S, Sp, G, s);
    return launch_t<T, NV, 2>(w, X, Y, rows, cols, row_bytes, S, Sp, G, s);
  } else if constexpr (NV == 2) {
    if (big && rows >= 256 * 4 * G) return launch_t<T, NV, 4>(w, X, Y, rows, cols, row_bytes, S, Sp, G, s);
    return launch_t<T, NV, 2>(w, X, Y, rows, cols, row_bytes, S, Sp, G, s);
  } else if constexpr (NV <= 8) {
    return launch_t<T, NV, 2>(w, X, Y, rows, cols, row_bytes, S, Sp, G, s);
  } else {
    return launch_t<T, NV, 1>(w, X, Y, rows, cols, row_bytes, S, Sp, G, s);
  }
}

template <uint32_t T>
static void launch_type(const void* w, const float* X, float* Y, int nvec, int rows, int cols, size_t row_bytes,
                        int S, int Sp, int G, hipStream_t s) {
  switch (nvec) {
    case 1: return launch_nv<T, 1>(w, X, Y, rows, cols, row_bytes, S, Sp, G, s);
    case 2: return launch_nv<T, 2>(w, X, Y, rows, cols, row_bytes, S, Sp, G, s);
    case 3: return launch_nv<T, 3>(w, X, Y, rows, cols, row_bytes, S, Sp, G, s);
    case 4: return launch_nv<T, 4>(w, X, Y, rows, cols, row_bytes, S, Sp, G, s);
    case 5: return launch_nv<T, 5>(w, X, Y, rows, cols, row_bytes, S, Sp, G, s);
    case 6: return launch_nv<T, 6>(w, X, Y, rows, cols, row_bytes, S, Sp, G, s);
    case 7: return launch_nv<T, 7>(w, X, Y, rows, cols, row_bytes, S, Sp, G, s);
    case 8: return launch_nv<T, 8>(w, X, Y, rows, cols, row_bytes, S, Sp, G, s);
    case 9: return launch_nv<T, 9>(w, X, Y, rows, cols, row_bytes, S, Sp, G, s);
    case 10: return launch_nv<T, 10>(w, X, Y, rows, cols, row_bytes, S, Sp, G, s);
    case 11: return launch_nv<T, 11>(w, X, Y, rows, cols, row_bytes, S, Sp, G, s);
    case 12: return launch_nv<T, 12>(w, X, Y, rows, cols, row_bytes, S, Sp, G, s);
    case 13: return launch_nv<T, 13>(w, X, Y, rows, cols, row_bytes, S, Sp, G, s);
    case 14: return launch_nv<T, 14>(w, X, Y, rows, cols, row_bytes, S, Sp, G, s);
    case 15: return launch_nv<T, 15>(w, X, Y, rows, cols, row_bytes, S, Sp, G, s);
    default: return launch_nv<T, 16>(w, X, Y, rows, cols, row_bytes, S, Sp, G, s);
  }
}

// Slot geometry of a row: S slots, padded group width Sp, groups per workgroup G.  Returns false
// when a row has more than 1024 slots (K > 32768): the generic kernel takes those.
bool gemv_geometry(uint32_t t, int cols, int& S, int& Sp, int& G) {
  const int spb = (t == T_Q4_K || t == T_Q6_K) ? 8 : 1;
  const int qk = (t == T_Q4_K || t == T_Q6_K) ? 256 : 32;
  S = cols / qk * spb;
  if (S <= 0 || S > 1024) return false;
  if (S <= 64) {
    Sp = 1;
    while (Sp < S) Sp <<= 1;
  } else {
    Sp = (S + 63) & ~63;
  }
  G = Sp >= 256 ? 1 : 256 / Sp;
  return true;
}

// Fast-path GEMV for 1 <= nvec <= 16 on 16-byte-aligned rows of Q8_0 / Q4_0 / Q4_K / Q6_K.
bool launch_gemv_fast(uint32_t t, const void* w, const float* X, float* Y, int nvec, int rows, int cols,
                      size_t row_bytes, hipStream_t s) {
  int S, Sp, G;
  if (!gemv_geometry(t, cols, S, Sp, G)) return false;
  switch (t) {
    case T_Q4_K: launch_type<T_Q4_K>(w, X, Y, nvec, rows, cols, row_bytes, S, Sp, G, s); return true;
    case T_Q6_K: launch_type<T_Q6_K>(w, X, Y, nvec, rows, cols, row_bytes, S, Sp, G, s); return true;
    case T_Q4_0: launch_type<T_Q4_0>(w, X, Y, nvec, rows, cols, row_bytes, S, Sp, G, s); return true;
    case T_Q8_0: launch_type<T_Q8_0>(w, X, Y, nvec, rows, cols, row_bytes, S, Sp, G, s); return true;
    default: return false;
  }
}

}  // namespace qvx
