// qvx_deq.hpp -- exact per-element dequantisation of the GGUF block formats (device code shared by
// the dequantise kernels and the prefill GEMM of the non-Q4_K types).  Every formula is the public
// ggml block definition as the reference states it in runtime/src/dequant.cpp:38-210; the products
// are exact in fp32, so the single rounding (Q4_K / Q5_K subtract, Q4_1 / Q5_1 add) gives the same
// value in any order.
#pragma once

#include "qvx_common.hpp"

namespace qvx {

__device__ inline uint32_t ld16(const uint8_t* p) { return (uint32_t)p[0] | ((uint32_t)p[1] << 8); }

__device__ inline void k4_scale_min(int j, const uint8_t* q, uint32_t& sc, uint32_t& m) {
  if (j < 4) {
    sc = q[j] & 63;
    m = q[j + 4] & 63;
  } else {
    sc = (q[j + 4] & 15) | ((q[j - 4] >> 6) << 4);
    m = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
  }
}

template <uint32_t T>
__device__ inline float deq_elem(const uint8_t* b, int e);

template <> __device__ inline float deq_elem<T_Q8_0>(const uint8_t* b, int e) {
  return f16_bits_to_f32(ld16(b)) * (float)(int8_t)b[2 + e];
}
template <> __device__ inline float deq_elem<T_Q8_1>(const uint8_t* b, int e) {
  return f16_bits_to_f32(ld16(b)) * (float)(int8_t)b[4 + e];
}
template <> __device__ inline float deq_elem<T_Q4_0>(const uint8_t* b, int e) {
  const int q = e < 16 ? (b[2 + e] & 15) : (b[2 + e - 16] >> 4);
  return (float)(q - 8) * f16_bits_to_f32(ld16(b));
}
template <> __device__ inline float deq_elem<T_Q4_1>(const uint8_t* b, int e) {
  const int q = e < 16 ? (b[4 + e] & 15) : (b[4 + e - 16] >> 4);
  return (float)q * f16_bits_to_f32(ld16(b)) + f16_bits_to_f32(ld16(b + 2));
}
template <> __device__ inline float deq_elem<T_Q5_0>(const uint8_t* b, int e) {
  const uint32_t qh = b[2] | (b[3] << 8) | (b[4] << 16) | ((uint32_t)b[5] << 24);
  const int lo = e < 16 ? (b[6 + e] & 15) : (b[6 + e - 16] >> 4);
  const int q = lo | (int)(((qh >> e) & 1u) << 4);
  return (float)(q - 16) * f16_bits_to_f32(ld16(b));
}
template <> __device__ inline float deq_elem<T_Q5_1>(const uint8_t* b, int e) {
  const uint32_t qh = b[4] | (b[5] << 8) | (b[6] << 16) | ((uint32_t)b[7] << 24);
  const int lo = e < 16 ? (b[8 + e] & 15) : (b[8 + e - 16] >> 4);
  const int q = lo | (int)(((qh >> e) & 1u) << 4);
  return (float)q * f16_bits_to_f32(ld16(b)) + f16_bits_to_f32(ld16(b + 2));
}
template <> __device__ inline float deq_elem<T_Q4_K>(const uint8_t* b, int e) {
  const int c = e >> 6, l = e & 63, hi = l >> 5;
  const uint8_t byte = b[16 + 32 * c + (l & 31)];
  const int nib = hi ? (byte >> 4) : (byte & 15);
  uint32_t sc, m;
  k4_scale_min(2 * c + hi, b + 4, sc, m);
  const float ds = f16_bits_to_f32(ld16(b)) * (float)sc;
  const float dm = f16_bits_to_f32(ld16(b + 2)) * (float)m;
  return ds * (float)nib - dm;
}
template <> __device__ inline float deq_elem<T_Q5_K>(const uint8_t* b, int e) {
  const int c = e >> 6, l = e & 63, hi = l >> 5;
  const uint8_t byte = b[48 + 32 * c + (l & 31)];
  int q = hi ? (byte >> 4) : (byte & 15);
  if (b[16 + (l & 31)] & (1u << (2 * c + hi))) q += 16;
  uint32_t sc, m;
  k4_scale_min(2 * c + hi, b + 4, sc, m);
  const float ds = f16_bits_to_f32(ld16(b)) * (float)sc;
  const float dm = f16_bits_to_f32(ld16(b + 2)) * (float)m;
  return ds * (float)q - dm;
}
template <> __device__ inline float deq_elem<T_Q6_K>(const uint8_t* b, int e) {
  const int h = e >> 7, p = e & 127, quarter = p >> 5, l = p & 31;
  const uint8_t* ql = b + 64 * h;
  const uint8_t* qh = b + 128 + 32 * h;
  const int8_t* sc = (const int8_t*)(b + 192 + 8 * h);
  const uint8_t lob = (quarter & 1) ? ql[l + 32] : ql[l];
  const int nib = (quarter & 2) ? (lob >> 4) : (lob & 15);
  const int q = nib | (((qh[l] >> (2 * quarter)) & 3) << 4);
  const float d = f16_bits_to_f32(ld16(b + 208));
  return d * (float)sc[(l >> 4) + 2 * quarter] * (float)(q - 32);
}
// F16 / BF16 have one element per 2-byte block, so e is always 0 here.
template <> __device__ inline float deq_elem<T_F16>(const uint8_t* b, int e) {
  return f16_bits_to_f32(ld16(b + 2 * e));
}
template <> __device__ inline float deq_elem<T_BF16>(const uint8_t* b, int e) {
  return __builtin_bit_cast(float, ld16(b + 2 * e) << 16);
}

}  // namespace qvx
