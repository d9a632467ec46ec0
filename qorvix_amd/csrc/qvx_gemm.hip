// qvx_gemm.hip -- prefill GEMM (M >= 128) over raw GGUF Q4_K blocks on gfx950 matrix cores.
//
// out[m, r] = sum_k X[m, k] * dequant(W)[r, k],  X fp16 [M, K], W Q4_K [N rows, K], out fp32 [M, N].
// No reference counterpart (the reference prefills token by token); the semantics are qmatmulN's
// (runtime/src/qmatmul.cpp:64-115) with X converted fp16 -> fp32 exactly.
//
// Tiling (256 threads = 4 waves, v_mfma_f32_32x32x16_{bf16,f16}):
//  * A workgroup computes a BM x (4*32*NT) output tile; wave w owns NT 32-row strips of W and
//    all BM tokens, so every weight element is dequantised exactly once per workgroup.
//  * K advances in slices of 64 elements = one 64-element group c of a Q4_K super-block.  Each
//    lane (n = lane%32, g = lane/32) loads the 16 quant bytes 32c+16g..+15 of its weight row and
//    the 16-byte super-block header straight into registers (aligned 16-byte loads), dequantises
//    them exactly in fp32 (d*sc*n - dmin*m, one rounding, the reference's dequant value), rounds to
//    bf16 / fp16 and uses them as the B operand of four K16 steps: low nibbles 0-7, 8-15, then high
//    nibbles 0-7, 8-15.  The A operand (X) is read from LDS in exactly that element order.
//  * The X slice (BM x 64 halves) is staged in a double-buffered LDS tile (row pitch padded by 16
//    bytes) with one barrier per slice; loads of slice k+1 are in flight during slice k's MFMAs.
//  * Small grids split K across workgroups and accumulate with fp32 atomics into a zeroed output.
#include "qvx_common.hpp"

namespace qvx {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef int i32x4_t __attribute__((ext_vector_type(4)));
typedef int i32x16_t __attribute__((ext_vector_type(16)));

enum { VAR_BF16 = 0, VAR_I8 = 1, VAR_F16 = 2 };

// Two fp32 -> one dword of two 16-bit values (round to nearest even).
template <int VAR> __device__ inline uint32_t pack2(float a, float b);
template <> __device__ inline uint32_t pack2<VAR_BF16>(float a, float b) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  bf16x2_t v = {(__bf16)a, (__bf16)b};
  return __builtin_bit_cast(uint32_t, v);
}
template <> __device__ inline uint32_t pack2<VAR_F16>(float a, float b) {
  half2_t v = {(_Float16)a, (_Float16)b};
  return __builtin_bit_cast(uint32_t, v);
}

// 6-bit (scale, min) of sub-blocks 2c, 2c+1 from a Q4_K header, as byte pairs (c uniform).
__device__ inline void q4k_pairs(const uint4& h, int c, uint32_t& scp, uint32_t& mp) {
  if (c < 2) {
    const uint32_t sh = 16u * (uint32_t)c;
    scp = (h.y >> sh) & 0x3F3Fu;
    mp = (h.z >> sh) & 0x3F3Fu;
  } else {
    const uint32_t sh = 16u * (uint32_t)(c - 2);
    scp = ((h.w >> sh) & 0x0F0Fu) | ((h.y >> (sh + 2)) & 0x3030u);
    mp = ((h.w >> (sh + 4)) & 0x0F0Fu) | ((h.z >> (sh + 2)) & 0x3030u);
  }
}

// Dequantises 8 nibbles (4 bytes of two dwords, low or high nibbles) to one MFMA operand.
template <int VAR>
__device__ inline i32x4_t deq8(uint32_t w0, uint32_t w1, float ds, float mdm) {
  i32x4_t o;
  o[0] = (int)pack2<VAR>(__builtin_fmaf(ds, (float)(w0 & 15u), mdm), __builtin_fmaf(ds, (float)((w0 >> 8) & 15u), mdm));
  o[1] = (int)pack2<VAR>(__builtin_fmaf(ds, (float)((w0 >> 16) & 15u), mdm), __builtin_fmaf(ds, (float)(w0 >> 24 & 15u), mdm));
  o[2] = (int)pack2<VAR>(__builtin_fmaf(ds, (float)(w1 & 15u), mdm), __builtin_fmaf(ds, (float)((w1 >> 8) & 15u), mdm));
  o[3] = (int)pack2<VAR>(__builtin_fmaf(ds, (float)((w1 >> 16) & 15u), mdm), __builtin_fmaf(ds, (float)(w1 >> 24 & 15u), mdm));
  return o;
}

template <int VAR>
__device__ inline f32x16_t mfma32(i32x4_t a, i32x4_t b, f32x16_t c) {
  if constexpr (VAR == VAR_BF16)
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b), c,
                                                   0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a), __builtin_bit_cast(f16x8_t, b), c, 0,
                                                  0, 0);
}

// X (fp16) -> the variant's 16-bit type, 8 values.
template <int VAR>
__device__ inline uint4 cvt_x8(uint4 v) {
  if constexpr (VAR == VAR_F16) {
    return v;
  } else {
    uint4 o;
    const uint32_t in[4] = {v.x, v.y, v.z, v.w};
    uint32_t r[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) r[i] = pack2<VAR_BF16>(f16lo(in[i]), f16hi(in[i]));
    o.x = r[0];
    o.y = r[1];
    o.z = r[2];
    o.w = r[3];
    return o;
  }
}

template <int VAR, int BM, int NT>
__global__ __launch_bounds__(256) void k_qgemm_q4k(const uint8_t* __restrict__ W, const uint16_t* __restrict__ X,
                                                   float* __restrict__ Y, int M, int N, int K, size_t row_bytes,
                                                   int slices_per_split, int atomic_out) {
  constexpr int MT = BM / 32;
  constexpr int BN = 4 * 32 * NT;
  constexpr int XS = 64 + 8;               // LDS row pitch in halves (144 bytes)
  constexpr int XCH = BM * 8;              // 16-byte chunks of one X slice
  constexpr int XLD = (XCH + 255) / 256;   // per thread
  __shared__ __attribute__((aligned(16))) uint16_t xl[2][BM * XS];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int ln = lane & 31, g = lane >> 5;
  const int m0 = blockIdx.y * BM;
  const int nw = blockIdx.x * BN + wave * 32 * NT;  // first weight row of this wave
  const int nsl = K / 64;
  const int kb0 = blockIdx.z * slices_per_split;
  const int kb1 = min(nsl, kb0 + slices_per_split);
  if (kb0 >= kb1) return;

  f32x16_t acc[MT][NT];
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int j = 0; j < NT; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

  uint4 xr[XLD];
  uint4 wq[NT], wh[NT];

  auto load_x = [&](int kb) {
#pragma unroll
    for (int j = 0; j < XLD; ++j) {
      const int q = tid + 256 * j;
      const int row = q >> 3, part = q & 7;
      uint4 v = {0u, 0u, 0u, 0u};
      if (q < XCH && m0 + row < M)
        v = *reinterpret_cast<const uint4*>(X + (size_t)(m0 + row) * K + (size_t)kb * 64 + 8 * part);
      xr[j] = v;
    }
  };
  auto store_x = [&](int buf) {
#pragma unroll
    for (int j = 0; j < XLD; ++j) {
      const int q = tid + 256 * j;
      const int row = q >> 3, part = q & 7;
      if (q < XCH) *reinterpret_cast<uint4*>(&xl[buf][row * XS + 8 * part]) = cvt_x8<VAR>(xr[j]);
    }
  };
  auto load_w = [&](int kb) {
    const int sb = kb >> 2, c = kb & 3;
#pragma unroll
    for (int j = 0; j < NT; ++j) {
      const int n = nw + 32 * j + ln;
      uint4 q = {0u, 0u, 0u, 0u}, h = {0u, 0u, 0u, 0u};
      if (n < N) {
        const uint8_t* blk = W + (size_t)n * row_bytes + (size_t)sb * 144;
        h = *reinterpret_cast<const uint4*>(blk);
        q = *reinterpret_cast<const uint4*>(blk + 16 + 32 * c + 16 * g);
      }
      wq[j] = q;
      wh[j] = h;
    }
  };

  load_x(kb0);
  load_w(kb0);
  store_x(0);
  for (int kb = kb0; kb < kb1; ++kb) {
    const int buf = (kb - kb0) & 1;
    __syncthreads();
    // B operands of this slice from the registers loaded one slice ago.
    i32x4_t bfrag[NT][4];
    const int c = kb & 3;
#pragma unroll
    for (int j = 0; j < NT; ++j) {
      uint32_t scp, mp;
      q4k_pairs(wh[j], c, scp, mp);
      const float d = f16lo(wh[j].x), dmin = f16hi(wh[j].x);
      const float ds0 = d * (float)(scp & 0xFFu), ds1 = d * (float)(scp >> 8);
      const float dm0 = -(dmin * (float)(mp & 0xFFu)), dm1 = -(dmin * (float)(mp >> 8));
      const uint32_t q0 = wq[j].x, q1 = wq[j].y, q2 = wq[j].z, q3 = wq[j].w;
      bfrag[j][0] = deq8<VAR>(q0, q1, ds0, dm0);
      bfrag[j][1] = deq8<VAR>(q2, q3, ds0, dm0);
      bfrag[j][2] = deq8<VAR>(q0 >> 4, q1 >> 4, ds1, dm1);
      bfrag[j][3] = deq8<VAR>(q2 >> 4, q3 >> 4, ds1, dm1);
    }
    if (kb + 1 < kb1) {
      load_x(kb + 1);
      load_w(kb + 1);
    }
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const int kof = 32 * (s >> 1) + 16 * g + 8 * (s & 1);
#pragma unroll
      for (int i = 0; i < MT; ++i) {
        const i32x4_t a = *reinterpret_cast<const i32x4_t*>(&xl[buf][(32 * i + ln) * XS + kof]);
#pragma unroll
        for (int j = 0; j < NT; ++j) acc[i][j] = mfma32<VAR>(a, bfrag[j][s], acc[i][j]);
      }
    }
    if (kb + 1 < kb1) store_x(buf ^ 1);
  }

  // C layout of v_mfma_f32_32x32x*: element e of lane l is row 8*(e/4) + 4*(l/32) + e%4, col l%32.
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int j = 0; j < NT; ++j) {
      const int n = nw + 32 * j + ln;
      if (n >= N) continue;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int m = m0 + 32 * i + 8 * (e >> 2) + 4 * g + (e & 3);
        if (m < M) {
          float* dst = Y + (size_t)m * N + n;
          if (atomic_out)
            unsafeAtomicAdd(dst, acc[i][j][e]);
          else
            *dst = acc[i][j][e];
        }
      }
    }
}

__global__ __launch_bounds__(256) void k_zero_f32(float* __restrict__ p, size_t n) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) p[i] = 0.0f;
}

// Zero fill by kernel (no memset nodes, so callers may capture it in a HIP graph).
void launch_zero(float* p, size_t n, hipStream_t s) {
  if (n) k_zero_f32<<<(unsigned)((n + 255) / 256), 256, 0, s>>>(p, n);
}

// ---- per-32 Q8 activation quantiser --------------------------------------------------------------
// One wave per (row, 64 blocks): lane = block of 32 values; fp32 math as the oracle states it.
__global__ __launch_bounds__(256) void k_quant_q8(const uint16_t* __restrict__ X, int M, int K, int8_t* __restrict__ q,
                                                  float* __restrict__ scale, int32_t* __restrict__ qsum) {
  const int nb = K / 32;
  const size_t blk = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (blk >= (size_t)M * nb) return;
  const uint16_t* x = X + blk * 32;
  float v[32];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint4 u = reinterpret_cast<const uint4*>(x)[i];
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      v[8 * i + 2 * j] = f16lo(w[j]);
      v[8 * i + 2 * j + 1] = f16hi(w[j]);
    }
  }
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < 32; ++i) amax = fmaxf(amax, fabsf(v[i]));
  const float s = amax / 127.0f;
  const float inv = amax > 0.0f ? 127.0f / amax : 0.0f;
  int sum = 0;
  uint32_t packed[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    uint32_t word = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float r = roundf(v[4 * i + j] * inv);
      r = fminf(fmaxf(r, -127.0f), 127.0f);
      const int qi = (int)r;
      sum += qi;
      word |= ((uint32_t)(qi & 0xFF)) << (8 * j);
    }
    packed[i] = word;
  }
  uint4* dst = reinterpret_cast<uint4*>(q + blk * 32);
  dst[0] = make_uint4(packed[0], packed[1], packed[2], packed[3]);
  dst[1] = make_uint4(packed[4], packed[5], packed[6], packed[7]);
  scale[blk] = s;
  qsum[blk] = sum;
}

int launch_quantize_act_q8(const uint16_t* X, int M, int K, int8_t* q, float* scale, int32_t* qsum, hipStream_t s) {
  if ((reinterpret_cast<uintptr_t>(X) & 15u) || (reinterpret_cast<uintptr_t>(q) & 15u)) return -7;  // QVX_E_RANGE
  const size_t nblk = (size_t)M * (K / 32);
  k_quant_q8<<<(unsigned)((nblk + 255) / 256), 256, 0, s>>>(X, M, K, q, scale, qsum);
  return 0;
}

template <int VAR, int BM, int NT>
static void launch_q4k(float* out, const void* w, const uint16_t* X, int M, int N, int K, hipStream_t s) {
  constexpr int BN = 4 * 32 * NT;
  const size_t row_bytes = (size_t)(K / 256) * 144;
  const int nsl = K / 64;
  const int tiles = ((N + BN - 1) / BN) * ((M + BM - 1) / BM);
  // Split K until the grid covers the 256 CUs about twice; each split keeps >= 8 slices.
  int splits = 1;
  while (tiles * splits < 512 && nsl / (splits * 2) >= 8) splits *= 2;
  const int per = (nsl + splits - 1) / splits;
  splits = (nsl + per - 1) / per;
  if (splits > 1) launch_zero(out, (size_t)M * N, s);
  dim3 grid((N + BN - 1) / BN, (M + BM - 1) / BM, splits);
  k_qgemm_q4k<VAR, BM, NT><<<grid, 256, 0, s>>>(static_cast<const uint8_t*>(w), X, out, M, N, K, row_bytes, per,
                                                 splits > 1 ? 1 : 0);
}

// Returns a QVX status (0 ok, -1 type, -7 range).
int launch_qgemm(float* out, const void* w, uint32_t t, const uint16_t* X, int M, int rows, int cols, int variant,
                 hipStream_t s) {
  if (t != T_Q4_K) return -1;
  if ((reinterpret_cast<uintptr_t>(w) & 15u) || (reinterpret_cast<uintptr_t>(X) & 15u)) return -7;
  if (variant == VAR_BF16) {
    launch_q4k<VAR_BF16, 128, 2>(out, w, X, M, rows, cols, s);
    return 0;
  }
  if (variant == VAR_F16) {
    launch_q4k<VAR_F16, 128, 2>(out, w, X, M, rows, cols, s);
    return 0;
  }
  return -1;  // the int8 variant is not built yet
}

}  // namespace qvx
