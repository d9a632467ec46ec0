// qvx_gemv_valu.hpp -- the VALU decode GEMV's arithmetic (slot layout, per-format lanes, the
// activation conversion) and its kernel body, shared by the standalone kernel (qvx_gemv.hip) and the
// grouped launch (qvx_gemv_mx.hip).  The design is described at the top of qvx_gemv.hip.
#pragma once

#include <algorithm>

#include "qvx_common.hpp"
#include "qvx_norm.hpp"

namespace qvx {

typedef uint32_t u32x4a4_t __attribute__((ext_vector_type(4), aligned(4)));  // dword-aligned 16 bytes
typedef short short2_t __attribute__((ext_vector_type(2)));

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

// High nibbles of four bytes in place, as signed bytes 16 (n - 8).
__device__ inline uint32_t hi_codes(uint32_t w) { return (w & 0xF0F0F0F0u) ^ 0x80808080u; }

// ---- activations of one slot in 15-bit fixed point --------------------------------------------
template <int R>
struct XQ {
  uint32_t h[4 * R], l[4 * R];  // qh / ql as signed bytes, 4 consecutive elements per dword; run r at [4r, 4r+4)
  int q[R];                     // sum of q over each run
  float sx;                     // x = q * sx (NaN when the slot holds a non-finite activation)
};
// LDS words per (vector, slot): h[4R], l[4R], q[R], sx, padded to a multiple of 4 words
template <int R>
constexpr int xq_words() {
  return (9 * R + 1 + 3) & ~3;
}

// sum(code * q) over N dwords of signed byte codes (4N elements).
template <int N>
__device__ inline int dotq(const uint32_t* c, const uint32_t* h, const uint32_t* l) {
  int s = 0;
#pragma unroll
  for (int j = 0; j < N; ++j) s = __builtin_amdgcn_sdot4((int)c[j], (int)h[j], s, false);
  s = (int)((uint32_t)s << 7);
#pragma unroll
  for (int j = 0; j < N; ++j) s = __builtin_amdgcn_sdot4((int)c[j], (int)l[j], s, false);
  return s;
}

// Per-type lane logic.  kR runs of 16 elements per slot; xoff(sig, r) = element offset of run r of
// slot sig within the row; Raw = the registers one row's slot needs; load() issues its global
// loads (rows are 16-byte aligned; offsets are row-relative); row() returns the slot's partial
// dot product with the activations, in units of sx.
template <uint32_t T> struct Lane;

// Q4_K: slot sig = scale group c = sig%4 (64 elements) of super-block b = sig/4: bytes 32c..32c+31
// of the 128 qs bytes; low nibbles are sub-block 2c (elements 64c + l, l = 0..31), high nibbles
// sub-block 2c+1 (elements 64c + 32 + l).  Runs: 0, 1 = sub-block 2c, 2, 3 = sub-block 2c+1.
template <> struct Lane<T_Q4_K> {
  static constexpr int kR = 4;
  static constexpr int kSlotElems = 64;
  struct Raw {
    uint4 h, q0, q1;
  };
  static __device__ inline int xoff(int sig, int run) { return 256 * (sig >> 2) + 64 * (sig & 3) + 16 * run; }
  static __device__ inline void load(const uint8_t* row, int sig, Raw& r) {
    const uint8_t* blk = row + 144 * (sig >> 2);
    r.h = ldg16(blk);
    r.q0 = ldg16(blk + 16 + 32 * (sig & 3));
    r.q1 = ldg16(blk + 32 + 32 * (sig & 3));
  }
  static __device__ inline float row(const Raw& r, int sig, const XQ<4>& x) {
    const uint32_t q[8] = {r.q0.x, r.q0.y, r.q0.z, r.q0.w, r.q1.x, r.q1.y, r.q1.z, r.q1.w};
    uint32_t lo[8], hi[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      lo[j] = q[j] & 0x0F0F0F0Fu;
      hi[j] = hi_codes(q[j]);
    }
    const int qa = x.q[0] + x.q[1], qb = x.q[2] + x.q[3];
    const int ta = dotq<8>(lo, x.h, x.l);                    // sum n q over sub-block 2c
    const int tb = dotq<8>(hi, x.h + 8, x.l + 8) + 128 * qb;  // 16 * sum n q over sub-block 2c+1
    // 6-bit (scale, min) of sub-blocks 2c, 2c+1 (public K-quant scale packing, scale bytes
    // s[0..11] = h.y, h.z, h.w): c < 2: sc = s[2c..2c+1] & 63, m = s[2c+4..] & 63; c >= 2: low 4
    // bits from s[2c+4..] (sc: low nibble, m: high nibble), high 2 bits from bits 6-7 of s[2c-4..]
    // (sc) and s[2c..] (m).  With j = 2(c%2): p1 = [y_j, y_j+1, z_j, z_j+1], p2 = [w_j, w_j+1,
    // w_j, w_j+1], and the packed result sm = [sc_a, sc_b, m_a, m_b].  Masks are lane-constant.
    const int c = sig & 3;
    const uint32_t j = 2u * (uint32_t)(c & 1);
    const uint32_t p1 = __builtin_amdgcn_perm(r.h.z, r.h.y, j | (j + 1) << 8 | (j + 4) << 16 | (j + 5) << 24);
    const uint32_t p2 = __builtin_amdgcn_perm(r.h.w, r.h.w, j | (j + 1) << 8 | j << 16 | (j + 1) << 24);
    const bool up = c >= 2;
    const uint32_t sm = (p1 & (up ? 0u : 0x3F3F3F3Fu)) | ((p1 >> 2) & (up ? 0x30303030u : 0u)) |
                        (p2 & (up ? 0x00000F0Fu : 0u)) | ((p2 >> 4) & (up ? 0x0F0F0000u : 0u));
    const float sca = (float)(sm & 0xFFu), scb = (float)((sm >> 8) & 0xFFu);  // v_cvt_f32_ubyte0..3
    const float mna = (float)((sm >> 16) & 0xFFu), mnb = (float)(sm >> 24);
    const float t = __builtin_fmaf((float)tb * 0.0625f, scb, (float)ta * sca);
    const float u = __builtin_fmaf((float)qb, mnb, (float)qa * mna);
    return __builtin_fmaf(f16lo(r.h.x), t, -f16hi(r.h.x) * u);
  }
};

// Q5_K (176-byte super-blocks: d, dmin, the Q4_K scale packing, qh[32], qs[128]): slot sig = scale
// group c = sig%4 of super-block b = sig/4, as for Q4_K, with qs at byte 48.  Element l of the
// group's low sub-block 2c is (qs[32c + l] & 15) + 16 * bit 2c of qh[l], of the high sub-block 2c+1
// (qs[32c + l] >> 4) + 16 * bit 2c+1 of qh[l] (public K-quant layout).  The 5-bit codes 0..31 are
// multiplied as they are, so no offset correction enters the fold.
template <> struct Lane<T_Q5_K> {
  static constexpr int kR = 4;
  static constexpr int kSlotElems = 64;
  struct Raw {
    uint4 h, qh0, qh1, q0, q1;
  };
  static __device__ inline int xoff(int sig, int run) { return 256 * (sig >> 2) + 64 * (sig & 3) + 16 * run; }
  static __device__ inline void load(const uint8_t* row, int sig, Raw& r) {
    const uint8_t* blk = row + 176 * (sig >> 2);
    r.h = ldg16(blk);
    r.qh0 = ldg16(blk + 16);
    r.qh1 = ldg16(blk + 32);
    r.q0 = ldg16(blk + 48 + 32 * (sig & 3));
    r.q1 = ldg16(blk + 64 + 32 * (sig & 3));
  }
  static __device__ inline float row(const Raw& r, int sig, const XQ<4>& x) {
    const uint32_t q[8] = {r.q0.x, r.q0.y, r.q0.z, r.q0.w, r.q1.x, r.q1.y, r.q1.z, r.q1.w};
    const uint32_t qh[8] = {r.qh0.x, r.qh0.y, r.qh0.z, r.qh0.w, r.qh1.x, r.qh1.y, r.qh1.z, r.qh1.w};
    const int c = sig & 3;
    const uint32_t sa = 2u * (uint32_t)c;  // bit of qh for the low sub-block; sa + 1 for the high
    uint32_t lo[8], hi[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const uint32_t ba = ((qh[j] >> sa) << 4) & 0x10101010u, bb = ((qh[j] >> (sa + 1u)) << 4) & 0x10101010u;
      lo[j] = __builtin_amdgcn_bitop3_b32(q[j], 0x0F0F0F0Fu, ba, 0xEA);          // (q & 15) | 16 h
      hi[j] = __builtin_amdgcn_bitop3_b32(q[j] >> 4, 0x0F0F0F0Fu, bb, 0xEA);
    }
    const int qa = x.q[0] + x.q[1], qb = x.q[2] + x.q[3];
    const int ta = dotq<8>(lo, x.h, x.l);          // sum n q over sub-block 2c
    const int tb = dotq<8>(hi, x.h + 8, x.l + 8);  // sum n q over sub-block 2c+1
    // scale / min of sub-blocks 2c, 2c+1: the Q4_K packing (see Lane<T_Q4_K>)
    const uint32_t j = 2u * (uint32_t)(c & 1);
    const uint32_t p1 = __builtin_amdgcn_perm(r.h.z, r.h.y, j | (j + 1) << 8 | (j + 4) << 16 | (j + 5) << 24);
    const uint32_t p2 = __builtin_amdgcn_perm(r.h.w, r.h.w, j | (j + 1) << 8 | j << 16 | (j + 1) << 24);
    const bool up = c >= 2;
    const uint32_t sm = (p1 & (up ? 0u : 0x3F3F3F3Fu)) | ((p1 >> 2) & (up ? 0x30303030u : 0u)) |
                        (p2 & (up ? 0x00000F0Fu : 0u)) | ((p2 >> 4) & (up ? 0x0F0F0000u : 0u));
    const float sca = (float)(sm & 0xFFu), scb = (float)((sm >> 8) & 0xFFu);
    const float mna = (float)((sm >> 16) & 0xFFu), mnb = (float)(sm >> 24);
    const float t = __builtin_fmaf((float)tb, scb, (float)ta * sca);
    const float u = __builtin_fmaf((float)qb, mnb, (float)qa * mna);
    return __builtin_fmaf(f16lo(r.h.x), t, -f16hi(r.h.x) * u);
  }
};

// Q6_K: slot = super-block b = sig/8, u = sig%8 -> half h = u/4, l-group t = (u/2)%2, e = u%2.
// Run 0 is quarter e (low nibbles of ql[64h + 32e + 16t ..+16]), run 1 quarter e+2 (their high
// nibbles), with 2-bit high parts from qh[32h + 16t ..+16], bits (2e, 2e+1) and (2e+4, 2e+5);
// scales sc[8h + t + 2e] and sc[8h + t + 2e + 4].  Super-blocks are 2-byte aligned: each 16-byte
// piece is read as a dword-aligned 16-byte window, completed by the 4-byte tail the lane of the next
// piece loaded (never past its super-block), and realigned.
template <> struct Lane<T_Q6_K> {
  static constexpr int kR = 2;
  static constexpr int kSlotElems = 32;
  // The 8 slots of a super-block sit on 8 consecutive lanes of one wave.  Each lane loads its ql and
  // qh pieces as dword-aligned 16-byte windows and one dword of the super-block's last 20 bytes
  // (scales and d); the 4-byte tails of its windows and its scale and d words are the first dwords
  // its block's other lanes loaded (exchange), so a row costs three vector loads a lane.
  struct Raw {
    u32x4a4_t l, h;
    uint32_t w;    // lane u of the block: dword min(u, 4) of the scale window
    uint32_t le, he, s0, s1, dd;  // filled by exchange
    uint32_t sh;   // byte misalignment of the pieces (0 or 2)
    uint32_t ssh;  // byte position of the first scale inside s0
  };
  static __device__ inline int xoff(int sig, int run) {
    const int u = sig & 7;
    return 256 * (sig >> 3) + 128 * (u >> 2) + 32 * (u & 1) + 16 * ((u >> 1) & 1) + 64 * run;
  }
  // Super-block b = sig / 8 starts at byte 210 b: its pieces are misaligned by sh = 2 (b odd) or 0.
  // Lane u = sig % 8 (half h, piece t, bit pair e) owns ql bytes [64h + 32e + 16t, +16) and qh
  // bytes [128 + 32h + 16t, +16); the scale window is [192 - sh, 208 - sh) in dwords 0..3 and
  // [206, 210) in dword 4, every byte inside the super-block.
  static __device__ inline void load(const uint8_t* row, int sig, Raw& r) {
    const int b = sig >> 3, u = sig & 7, h = u >> 2, t = (u >> 1) & 1, e = u & 1;
    const int base = 210 * b, sh = base & 3;
    const int ol = base + 64 * h + 32 * e + 16 * t, oh = base + 128 + 32 * h + 16 * t;
    r.sh = (uint32_t)sh;
    r.l = ldg16a4(row + ol - sh);
    r.h = ldg16a4(row + oh - sh);
    r.w = ldg4(row + (u < 4 ? base + 192 - sh + 4 * u : base + 206));
  }
  // The words a lane takes from its block's lanes (bl: wave lane of the block's slot 0; padding
  // lanes pass the block of the slot they mirror).  le: the first dword after the ql window, the
  // next ql piece's (the piece at 128 is lane 0's qh window); he: the next qh piece's (after the
  // last one, scale dword 0); s0, s1: the dwords holding scale i = 8h + t + 2e and i + 4; dd: d.
  static __device__ inline void exchange(Raw& r, int sig, int bl) {
    const int u = sig & 7, h = u >> 2, t = (u >> 1) & 1, e = u & 1;
    const int nl = 64 * h + 32 * e + 16 * t + 16, nh = 32 * h + 16 * t + 16;
    const int ul = nl == 128 ? 0 : 4 * (nl >> 6) + 2 * ((nl >> 4) & 1) + ((nl >> 5) & 1);
    const int uh = nh == 64 ? 0 : 4 * (nh >> 5) + 2 * ((nh >> 4) & 1);
    const int pl = (int)(u == 0 ? r.h.x : r.l.x), ph = (int)(u == 0 ? r.w : r.h.x);
    const int si = (int)r.sh + 8 * h + t + 2 * e, q = si >> 2, ab = 4 * bl;
    r.le = (uint32_t)__builtin_amdgcn_ds_bpermute(ab + 4 * ul, pl);
    r.he = (uint32_t)__builtin_amdgcn_ds_bpermute(ab + 4 * uh, ph);
    r.s0 = (uint32_t)__builtin_amdgcn_ds_bpermute(ab + 4 * q, (int)r.w);
    r.s1 = (uint32_t)__builtin_amdgcn_ds_bpermute(ab + 4 * (q + 1), (int)r.w);
    r.dd = (uint32_t)__builtin_amdgcn_ds_bpermute(ab + 16, (int)r.w) >> 16;
    r.ssh = (uint32_t)(si & 3);
  }
  static __device__ inline float row(const Raw& r, int sig, const XQ<2>& x) {
    const uint32_t e = (uint32_t)(sig & 1);
    uint32_t ql[4], qh[4], a[4], b[4];
    realign16(r.l, r.le, r.sh, ql);
    realign16(r.h, r.he, r.sh, qh);
    const uint32_t shl = 4u - 2u * e, shr = 2u * e;
#pragma unroll
    for (int j = 0; j < 4; ++j) {  // 6-bit codes 0..63
      a[j] = (ql[j] & 0x0F0F0F0Fu) | ((qh[j] << shl) & 0x30303030u);         // bits (2e, 2e+1) -> 4..5
      b[j] = ((ql[j] >> 4) & 0x0F0F0F0Fu) | ((qh[j] >> shr) & 0x30303030u);  // bits (2e+4, 2e+5) -> 4..5
    }
    const int ta = dotq<4>(a, x.h, x.l) - 32 * x.q[0];  // sum (code - 32) q, exact in int32
    const int tb = dotq<4>(b, x.h + 4, x.l + 4) - 32 * x.q[1];
    // sc[.. + 4] is 4 bytes later: same byte position in the next dword.  The builtin's result
    // type is unsigned: the (int) keeps the conversion signed.
    const float sa = (float)(int)__builtin_amdgcn_sbfe((int)r.s0, 8u * r.ssh, 8u);
    const float sb = (float)(int)__builtin_amdgcn_sbfe((int)r.s1, 8u * r.ssh, 8u);
    return fold(f16lo(r.dd), sa, sb, ta, tb);
  }
  // The slot's partial from its two exact run sums (sum (code - 32) q per run): shared with the
  // batched matrix-core form, so both evaluate the same float operations.
  static __device__ inline float fold(float d, float sa, float sb, int ta, int tb) {
    return d * __builtin_fmaf(sb, (float)tb, sa * (float)ta);
  }
};

// Q4_0: slot sig = blocks 2 sig, 2 sig + 1 (36 bytes at 36 sig, dword aligned): block k holds its
// fp16 scale at bytes 18k..18k+1 and qs at 18k+2..18k+17; low nibbles of qs[i] are element i,
// high nibbles element 16 + i.  Runs: 0, 1 = block 0 (low, high), 2, 3 = block 1.
template <> struct Lane<T_Q4_0> {
  static constexpr int kR = 4;
  static constexpr int kSlotElems = 64;
  struct Raw {
    u32x4a4_t a, b;
    uint32_t e;
  };
  static __device__ inline int xoff(int sig, int run) { return 64 * sig + 16 * run; }
  static __device__ inline void load(const uint8_t* row, int sig, Raw& r) {
    const uint8_t* p = row + 36 * sig;
    r.a = ldg16a4(p);
    r.b = ldg16a4(p + 16);
    r.e = ldg4(p + 32);
  }
  // 16 * sum((n - 8) q) over one block
  static __device__ inline int block(const uint32_t (&qs)[4], const uint32_t* h, const uint32_t* l, int q_lo) {
    uint32_t lo[4], hi[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      lo[j] = qs[j] & 0x0F0F0F0Fu;
      hi[j] = hi_codes(qs[j]);
    }
    return 16 * dotq<4>(lo, h, l) + dotq<4>(hi, h + 4, l + 4) - 128 * q_lo;
  }
  static __device__ inline float row(const Raw& r, int, const XQ<4>& x) {
    const uint32_t q0[4] = {align_bytes(r.a.y, r.a.x, 2), align_bytes(r.a.z, r.a.y, 2), align_bytes(r.a.w, r.a.z, 2),
                            align_bytes(r.b.x, r.a.w, 2)};
    const uint32_t q1[4] = {r.b.y, r.b.z, r.b.w, r.e};
    const int v0 = block(q0, x.h, x.l, x.q[0]);
    const int v1 = block(q1, x.h + 8, x.l + 8, x.q[2]);
    return 0.0625f * __builtin_fmaf(f16hi(r.b.x), (float)v1, f16lo(r.a.x) * (float)v0);
  }
};

// Q5_0: slot sig = blocks 2 sig, 2 sig + 1 (44 bytes at 44 sig, dword aligned): block k holds its
// fp16 scale at bytes 22k..22k+1, the fifth bits qh (bit i for element i) at 22k+2..22k+5 and qs at
// 22k+6..22k+21; element i < 16 is (qs[i] & 15) + 16 * bit i, element 16 + i is (qs[i] >> 4) +
// 16 * bit (16 + i), value d * (code - 16) (dequant.cpp:75-91).  Runs as for Q4_0.  Codes 0..31
// are multiplied as they are and 16 * sum q subtracted per block.
template <> struct Lane<T_Q5_0> {
  static constexpr int kR = 4;
  static constexpr int kSlotElems = 64;
  struct Raw {
    u32x4a4_t a, b;
    uint32_t c0, c1, c2;
  };
  static __device__ inline int xoff(int sig, int run) { return 64 * sig + 16 * run; }
  static __device__ inline void load(const uint8_t* row, int sig, Raw& r) {
    const uint8_t* p = row + 44 * sig;
    r.a = ldg16a4(p);
    r.b = ldg16a4(p + 16);
    r.c0 = ldg4(p + 32);
    r.c1 = ldg4(p + 36);
    r.c2 = ldg4(p + 40);
  }
  // byte k of the result = 16 * bit k of the low four bits of n
  static __device__ inline uint32_t spread4(uint32_t n) { return (__umul24(n & 15u, 0x00204081u) & 0x01010101u) << 4; }
  // sum((code - 16) q) over one block: quant dwords qs, fifth bits qh
  static __device__ inline int block(const uint32_t (&qs)[4], uint32_t qh, const uint32_t* h, const uint32_t* l,
                                     int q_lo, int q_hi) {
    uint32_t lo[4], hi[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      lo[j] = (qs[j] & 0x0F0F0F0Fu) | spread4(qh >> (4 * j));
      hi[j] = ((qs[j] >> 4) & 0x0F0F0F0Fu) | spread4(qh >> (16 + 4 * j));
    }
    return dotq<4>(lo, h, l) + dotq<4>(hi, h + 4, l + 4) - 16 * (q_lo + q_hi);
  }
  static __device__ inline float row(const Raw& r, int, const XQ<4>& x) {
    const uint32_t w[11] = {r.a.x, r.a.y, r.a.z, r.a.w, r.b.x, r.b.y, r.b.z, r.b.w, r.c0, r.c1, r.c2};
    const uint32_t qh0 = align_bytes(w[1], w[0], 2);  // bytes 2..5
    const uint32_t q0[4] = {align_bytes(w[2], w[1], 2), align_bytes(w[3], w[2], 2), align_bytes(w[4], w[3], 2),
                            align_bytes(w[5], w[4], 2)};  // bytes 6..21
    const uint32_t q1[4] = {w[7], w[8], w[9], w[10]};   // bytes 28..43
    const int v0 = block(q0, qh0, x.h, x.l, x.q[0], x.q[1]);
    const int v1 = block(q1, w[6], x.h + 8, x.l + 8, x.q[2], x.q[3]);
    return __builtin_fmaf(f16hi(w[5]), (float)v1, f16lo(w[0]) * (float)v0);
  }
};

// Q8_0: slot sig = blocks 2 sig, 2 sig + 1 (68 bytes at 68 sig, dword aligned): block k holds its
// fp16 scale at bytes 34k..34k+1 and 32 signed codes at 34k+2..34k+33.  Runs 0, 1 = block 0.
template <> struct Lane<T_Q8_0> {
  static constexpr int kR = 4;
  static constexpr int kSlotElems = 64;
  struct Raw {
    u32x4a4_t a, b, c, d;
    uint32_t e;
  };
  static __device__ inline int xoff(int sig, int run) { return 64 * sig + 16 * run; }
  static __device__ inline void load(const uint8_t* row, int sig, Raw& r) {
    const uint8_t* p = row + 68 * sig;
    r.a = ldg16a4(p);
    r.b = ldg16a4(p + 16);
    r.c = ldg16a4(p + 32);
    r.d = ldg16a4(p + 48);
    r.e = ldg4(p + 64);
  }
  static __device__ inline float row(const Raw& r, int, const XQ<4>& x) {
    const uint32_t w[17] = {r.a.x, r.a.y, r.a.z, r.a.w, r.b.x, r.b.y, r.b.z, r.b.w, r.c.x,
                            r.c.y, r.c.z, r.c.w, r.d.x, r.d.y, r.d.z, r.d.w, r.e};
    uint32_t q0[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) q0[j] = align_bytes(w[j + 1], w[j], 2);  // bytes 2..33
    const int t0 = dotq<8>(q0, x.h, x.l);
    const int t1 = dotq<8>(w + 9, x.h + 8, x.l + 8);  // bytes 36..67
    return __builtin_fmaf(f16hi(w[8]), (float)t1, f16lo(w[0]) * (float)t0);
  }
};

// ---- cross-lane sums (every lane of the span ends with the same bits: only commutative adds) --
template <int CTRL>
__device__ inline float dpp(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
template <int CTRL>
__device__ inline int dpp(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}
constexpr int kXor1 = 0xB1, kXor2 = 0x4E;            // quad_perm [1,0,3,2] / [2,3,0,1]
constexpr int kHalfMirror = 0x141, kMirror = 0x140;  // lane i <-> 7-i of 8 / 15-i of 16

// Sum over aligned spans of `width` lanes (8, 16, 32 or 64).
__device__ inline float span_sum(float s, int width) {
  s += dpp<kXor1>(s);
  s += dpp<kXor2>(s);
  s += dpp<kHalfMirror>(s);
  if (width > 8) s += dpp<kMirror>(s);
  if (width > 16) {  // rows of 16: swap odd rows of one copy with even rows of the other
    const auto a = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(int, s), __builtin_bit_cast(int, s), false, false);
    s = __builtin_bit_cast(float, (int)a[0]) + __builtin_bit_cast(float, (int)a[1]);
  }
  if (width > 32) {  // halves of the wave
    const auto a = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(int, s), __builtin_bit_cast(int, s), false, false);
    s = __builtin_bit_cast(float, (int)a[0]) + __builtin_bit_cast(float, (int)a[1]);
  }
  return s;
}

// ---- activation conversion (whole workgroup, into LDS) ---------------------------------------
// A task converts 8 elements: half `hf` of run `run` of (vector, slot) vs, task t = 2R vs + 2 run + hf.
// The 2R tasks of a slot are 2R aligned lanes of one wave (blockDim is a multiple of 8).  A
// thread's tasks are t = tid + k*blockDim (k < TPT); tasks past the end are clamped to the last
// (same data, results not stored) so every load is unconditional.
template <uint32_t T, int NV>
__device__ inline const float* task_x(const float* X, int cols, int S, int t) {
  using L = Lane<T>;
  static_assert(NV >= 1 && NV <= 4, "one to four vectors per launch");
  constexpr int R = L::kR;
  const int vs = t / (2 * R), part = t % (2 * R);
  const int v = NV == 1 ? 0 : vs / S, s = vs - v * S;
  return X + (size_t)v * cols + L::xoff(s, part >> 1) + 8 * (part & 1);
}

template <int R>
__device__ inline void convert_task(const float4 x0, const float4 x1, int t, bool store, uint32_t* xs,
                                    float* sx_out = nullptr) {
  const int vs = t / (2 * R), part = t % (2 * R), run = part >> 1, hf = part & 1;
  float a = fmaxf(fmaxf(fmaxf(fabsf(x0.x), fabsf(x0.y)), fmaxf(fabsf(x0.z), fabsf(x0.w))),
                  fmaxf(fmaxf(fabsf(x1.x), fabsf(x1.y)), fmaxf(fabsf(x1.z), fabsf(x1.w))));
  // 0 when the eight elements are finite, NaN otherwise (x * 0 is NaN for +-Inf and NaN)
  float z = __builtin_fmaf(x0.x, 0.0f, __builtin_fmaf(x0.y, 0.0f, __builtin_fmaf(x0.z, 0.0f, x0.w * 0.0f)));
  z = __builtin_fmaf(x1.x, 0.0f, __builtin_fmaf(x1.y, 0.0f, __builtin_fmaf(x1.z, 0.0f, __builtin_fmaf(x1.w, 0.0f, z))));
  a = fmaxf(a, dpp<kXor1>(a));
  a = fmaxf(a, dpp<kXor2>(a));
  z += dpp<kXor1>(z);
  z += dpp<kXor2>(z);
  if constexpr (R == 4) {
    a = fmaxf(a, dpp<kHalfMirror>(a));
    z += dpp<kHalfMirror>(z);
  }
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
  sq += dpp<kXor1>(sq);  // the other half of the run
  if (store) {
    uint32_t* o = xs + (size_t)vs * xq_words<R>();
    const int w = 4 * run + 2 * hf;
    o[w] = __builtin_amdgcn_perm(hs[1], hs[0], 0x06040200u);  // low bytes of the four 16-bit lanes
    o[w + 1] = __builtin_amdgcn_perm(hs[3], hs[2], 0x06040200u);
    o[4 * R + w] = __builtin_amdgcn_perm(ls[1], ls[0], 0x06040200u);
    o[4 * R + w + 1] = __builtin_amdgcn_perm(ls[3], ls[2], 0x06040200u);
    if (hf == 0) o[8 * R + run] = (uint32_t)sq;
    if (part == 0) o[9 * R] = __builtin_bit_cast(uint32_t, a * (1.0f / 16383.0f) + z);
    if (part == 0 && sx_out) *sx_out = a * (1.0f / 16383.0f) + z;
  }
}

template <int R>
__device__ inline void read_xq(const uint32_t* xs, XQ<R>& x) {
  const uint4* p = reinterpret_cast<const uint4*>(xs);
#pragma unroll
  for (int i = 0; i < R; ++i) {
    const uint4 h = p[i], l = p[R + i];
    x.h[4 * i] = h.x; x.h[4 * i + 1] = h.y; x.h[4 * i + 2] = h.z; x.h[4 * i + 3] = h.w;
    x.l[4 * i] = l.x; x.l[4 * i + 1] = l.y; x.l[4 * i + 2] = l.z; x.l[4 * i + 3] = l.w;
  }
  if constexpr (R == 2) {
    const uint4 m = p[4];
    x.q[0] = (int)m.x;
    x.q[1] = (int)m.y;
    x.sx = __uint_as_float(m.z);
  } else {
    const uint4 m = p[8];
    x.q[0] = (int)m.x;
    x.q[1] = (int)m.y;
    x.q[2] = (int)m.z;
    x.q[3] = (int)m.w;
    x.sx = __builtin_bit_cast(float, xs[36]);
  }
}

// Dynamic LDS bytes of the kernel: the converted activations.
template <uint32_t T>
inline size_t gemv_lds_bytes(int nv, int S) {
  return (size_t)nv * S * xq_words<Lane<T>::kR>() * 4;
}

// Launch geometry: blockDim = (Sp, G); workgroup b owns rows [rb, rb + cnt) with
// rb = b*base + min(b, rem), cnt = base + (b < rem).
struct Geo {
  int S, Sp, G;
  int base, rem;
  uint32_t row_bytes;
};

// One workgroup: G groups of Sp lanes; group g computes rows rb + g + G*i (g + G*i < cnt), RMAX rows
// a chunk, so one workgroup per CU can stream any number of rows after converting the activations
// once.
// TPT = conversion tasks per thread (NV * S * 2R <= TPT * blockDim).  Every global load is issued
// unconditionally (rows past the workgroup's last are clamped to it and their results dropped):
// activations first, then the first PF rows, and each later row PF rows ahead of its use, so a
// row's arithmetic waits only for its own bytes while the next ones are arriving.
// NORM: the activations are rmsnorm(x, NW, eps), folded into the conversion (cols % 512 == 0).
// Threads of a workgroup: 1024, or 512 for four vectors of the formats other than Q6_K, whose four
// vectors' fixed-point activations need more registers than a wave may hold at 16 waves a CU.  The
// per-vector arithmetic does not depend on how many groups a workgroup holds.
template <uint32_t T, int NV>
constexpr int gemv_threads() {
  return NV == 4 && T != T_Q6_K ? 512 : 1024;
}

// The kernel's body, for workgroup b with lane sig0 of group g (the standalone kernel passes
// blockIdx.x and its 2-D thread index; a grouped launch passes its own block numbering).
template <uint32_t T, int NV, int RMAX, int TPT, int PF, bool CH, bool NORM>
__device__ __forceinline__ void gemv_valu_body(const uint8_t* __restrict__ W, const float* __restrict__ X,
                                               float* __restrict__ Y, int rows, int cols, const Geo& geo,
                                               const float* __restrict__ NW, float eps, int b, int sig0, int g) {
  using L = Lane<T>;
  constexpr int R = L::kR;
  extern __shared__ uint4 xs_lds[];
  __shared__ float red[16][16];  // [output of the group][wave of the group] for groups wider than a wave
  __shared__ __attribute__((aligned(16))) float sqp[NORM ? NV * kNormMaxChunks : 4];  // chunk sums of squares
  uint32_t* xs = reinterpret_cast<uint32_t*>(xs_lds);
  const int S = geo.S, Sp = geo.Sp, G = geo.G;
  const int tid = g * Sp + sig0, nthr = Sp * G;
  const int sig = min(sig0, S - 1);  // padding lanes mirror the last slot; their partials are zeroed
  const int rb = b * geo.base + min(b, geo.rem), cnt = geo.base + (b < geo.rem ? 1 : 0);
  const uint8_t* wb = W + (size_t)rb * geo.row_bytes;
  const int ntask = NV * S * 2 * R;

  // 1. activations of this thread's conversion tasks (and, with NORM, the norm weights beside them)
  float4 xr[TPT][2], wr[TPT][2];
#pragma unroll
  for (int k = 0; k < TPT; ++k) {
    const float* px = task_x<T, NV>(X, cols, S, min(tid + k * nthr, ntask - 1));
    const float4* p = reinterpret_cast<const float4*>(px);
    xr[k][0] = p[0];
    xr[k][1] = p[1];
    if constexpr (NORM) {
      const float4* q = reinterpret_cast<const float4*>(NW + ((px - X) % cols));
      wr[k][0] = q[0];
      wr[k][1] = q[1];
    }
  }

  // 2. the quant bytes of the first PF rows (row offsets within the workgroup fit 32 bits)
  typename L::Raw raw[PF];
#pragma unroll
  for (int i = 0; i < PF; ++i) L::load(wb + (uint32_t)min(g + G * i, cnt - 1) * geo.row_bytes, sig, raw[i]);
  __builtin_amdgcn_sched_barrier(0);  // keep the loads here: the scheduler would sink them to their uses

  // 3. (NORM) each vector's sum of squares in the engine's canonical order (512-element chunks,
  // lane i of a chunk's wave summing elements 8i .. 8i+7; this kernel's conversion tasks are not in
  // element order, so the chunks are read again, from L2), every task scaled by its vector's factor;
  // then fixed-point activations into LDS
  if constexpr (NORM) {
    const int wave = tid >> 6, lane = tid & 63, nw = nthr >> 6, nch = cols / kNormChunk;
    const uint32_t sq_base = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) float*)sqp;
    for (int q = wave; q < NV * nch; q += nw) {
      const int v = q / nch, c = q - v * nch;
      const float4* p = reinterpret_cast<const float4*>(X + (size_t)v * cols + kNormChunk * c + 8 * lane);
      const float sq = wave_sum64(norm_sq8(p[0], p[1]));
      if (lane == 0) norm_store(sq_base + 4u * (uint32_t)(v * kNormMaxChunks + c), sq);
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
    __builtin_amdgcn_s_barrier();
    const int per = S * 2 * R;
#pragma unroll
    for (int k = 0; k < TPT; ++k) {
      const int v = min(tid + k * nthr, ntask - 1) / per;
      const float scale = norm_scale(sq_base + 4u * (uint32_t)(v * kNormMaxChunks), nch, cols, eps);
      norm_apply(xr[k][0], xr[k][1], scale, wr[k][0], wr[k][1]);
    }
  }
#pragma unroll
  for (int k = 0; k < TPT; ++k) {
    const int t = tid + k * nthr;
    convert_task<R>(xr[k][0], xr[k][1], min(t, ntask - 1), t < ntask, xs);
  }
  __syncthreads();

  // 4. rows in arrival order, RMAX at a time; each chunk is reduced and written before the next.
  // CH (several chunks): the loads run PF rows ahead across chunk boundaries (RMAX is a multiple of
  // PF, so row i always lands in raw[i % PF]); like every row load they are unconditional, the last
  // chunk's PF look-ahead loads re-reading the last row.  Without CH there is one chunk and no
  // load past it.
  XQ<R> x[NV];
#pragma unroll
  for (int v = 0; v < NV; ++v) read_xq<R>(xs + ((size_t)v * S + sig) * xq_words<R>(), x[v]);
  const float keep = sig0 < S ? 1.0f : 0.0f;
  // wave lane of the first slot of this lane's super-block (a group starts at a multiple of 8 lanes,
  // and its padding lanes share the wave of its last slot, whose block they mirror)
  const int blane = (g * Sp + (sig & ~7)) & 63;
  static_assert(!CH || RMAX % PF == 0, "chunks keep the prefetch ring aligned");
  const int nchunk = CH ? ((cnt + G - 1) / G + RMAX - 1) / RMAX : 1;  // the same for every group
  for (int c = 0; c < nchunk; ++c) {
    const int i0 = c * RMAX;
    float p[RMAX][NV];
#pragma unroll
    for (int i = 0; i < RMAX; ++i) {
      if constexpr (T == T_Q6_K) L::exchange(raw[i % PF], sig, blane);
#pragma unroll
      for (int v = 0; v < NV; ++v) {
        p[i][v] = L::row(raw[i % PF], sig, x[v]) * (x[v].sx * keep);
        // the product is rounded before the lane sums add it (no fused multiply-add into them), the
        // arithmetic the batched matrix-core form reproduces
        asm volatile("" : "+v"(p[i][v]));
      }
      if (CH || i + PF < RMAX)
        L::load(wb + (uint32_t)min(g + G * (i0 + i + PF), cnt - 1) * geo.row_bytes, sig, raw[i % PF]);
      __builtin_amdgcn_sched_barrier(0);
    }

    // 5. reduction over the group's S' lanes (fixed order)
    if (Sp <= 64) {
#pragma unroll
      for (int i = 0; i < RMAX; ++i) {
        const int r = g + G * (i0 + i);
#pragma unroll
        for (int v = 0; v < NV; ++v) {
          const float s = span_sum(p[i][v], Sp);
          if (sig0 == 0 && r < cnt) Y[(size_t)v * rows + rb + r] = s;
        }
      }
    } else {
      const int wig = sig0 >> 6, nw = Sp >> 6;  // wave index within the group, waves per group
      // outputs in chunks of 16 so the LDS table stays small for any RMAX * NV
      constexpr int NO = RMAX * NV;
#pragma unroll
      for (int o0 = 0; o0 < NO; o0 += 16) {
#pragma unroll
        for (int o = o0; o < NO && o < o0 + 16; ++o) {
          const float s = span_sum(p[o / NV][o % NV], 64);
          if ((sig0 & 63) == 0) red[o - o0][g * nw + wig] = s;
        }
        __syncthreads();
        // one thread per (group, output): sum the group's wave partials in wave order
        const int gg = tid >> 4, oo = tid & 15;
        if (gg < G && o0 + oo < NO) {
          const int i = (o0 + oo) / NV, v = (o0 + oo) % NV;
          const int r = gg + G * (i0 + i);
          if (r < cnt) {
            float s = 0.0f;
            for (int w = 0; w < nw; ++w) s += red[oo][gg * nw + w];
            Y[(size_t)v * rows + rb + r] = s;
          }
        }
        __syncthreads();
      }
    }
  }
}


// ---- launch geometry (the standalone launcher in qvx_gemv.hip and the grouped launch share it) ---

constexpr int kCUs = 256;  // MI355X compute units

// Rows a group keeps in flight ahead of the one being computed (measured per type: the 6-bit
// formats, with the most registers per row, do best with one, Q6_K two when a launch takes one
// vector; deeper rings spill with more vectors).
template <uint32_t T, int NV>
constexpr int prefetch_rows() {
  return T == T_Q6_K ? (NV == 1 ? 2 : 1) : T == T_Q5_K ? 1 : 2;
}

// Most rows a group takes (its partial sums stay in registers until the end).
template <int NV, int TPT>
constexpr int max_rows() {
  return NV == 1 && TPT < 8 ? 8 : 4;
}

// Slot geometry of a row: S slots, padded group width Sp, groups per workgroup G.  Returns false
// when K is not a whole number of slots, a row has more than 1024 slots, or two vectors'
// converted activations do not fit in LDS: the generic kernel takes those.
template <uint32_t T>
inline bool geometry(int cols, size_t row_bytes, Geo& geo) {
  constexpr int E = Lane<T>::kSlotElems;
  if (cols % E != 0 || row_bytes > 0xFFFFFFFFull / 1024) return false;
  const int S = cols / E;
  if (S <= 0 || S > 1024 || gemv_lds_bytes<T>(2, S) > 150 * 1024) return false;
  int Sp;
  if (S <= 64) {
    Sp = 8;
    while (Sp < S) Sp <<= 1;
  } else {
    Sp = (S + 63) & ~63;
  }
  geo.S = S;
  geo.Sp = Sp;
  geo.G = 1024 / Sp;
  geo.row_bytes = (uint32_t)row_bytes;
  return true;
}

// Grid over `rows` rows for geometry geo (S, Sp, G set): one pass of workgroups over the chip
// (16 waves per CU), at least one row per group on average.  Sets geo.base / geo.rem and the most
// rows a group takes (a group with more than max_rows walks them in chunks); returns the
// workgroup count.
inline int valu_grid(int rows, Geo& geo, int& per_group) {
  const int G = geo.G, waves = geo.Sp * G / 64;
  int64_t nwg = (int64_t)kCUs * (waves >= 16 ? 1 : 16 / waves);
  nwg = std::min<int64_t>(nwg, ((int64_t)rows + G - 1) / G);
  geo.base = (int)(rows / nwg);
  geo.rem = (int)(rows % nwg);
  per_group = (geo.base + (geo.rem ? 1 : 0) + G - 1) / G;
  return (int)nwg;
}

}  // namespace qvx
