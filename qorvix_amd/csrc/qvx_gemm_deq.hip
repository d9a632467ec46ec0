// qvx_gemm_deq.hip -- prefill GEMM of Q6_K weights whose rows hold an odd number of blocks (rows of
// an even number, W dword aligned, take k_qgemm_q6k8 in qvx_gemm.hip; Q4_K has its own kernels
// there): the raw blocks of each half super-block are staged in LDS for the tile's 256 weight rows,
// each row's 64-element K slices are dequantised from there into a 16-bit B tile in LDS, then
// bf16 / fp16 MFMA.
//
// out[m, r] = sum_k X[m, k] * dequant(W)[r, k],  X [M, K] 16-bit, W raw GGUF blocks [N rows, K],
// out fp32 [M, N].  No reference counterpart (the reference prefills token by token); the semantics
// are qmatmulN's (runtime/src/qmatmul.cpp:64-115) with X converted fp16 -> fp32 exactly.  Each
// weight element is the reference's exact dequantised value (runtime/src/dequant.cpp:164-191)
// rounded once to bf16 / fp16.
//
// Workgroup = 512 threads (8 waves, two per SIMD) computing a 128-token x 256-row tile; wave w owns
// tokens 64 (w % 2) .. +63 and weight rows 64 (w / 2) .. +63: 2 x 2 tiles of
// v_mfma_f32_32x32x16_{bf16,f16} (acc in registers).  Waves 0-3 also dequantise (thread t: tile row
// t), so one wave's VALU runs beside the other's MFMAs on each SIMD.  K advances in slices of 64 (a
// quarter of a Q6_K super-block; slices 2hb and 2hb + 1 form half super-block hb).  LDS (160 KiB):
//  * X stages (2 x 16 KiB): the slice's 128 token rows x 128 bytes, copied global -> LDS by
//    buffer_load ... lds one slice ahead;
//  * raw stages (2 x 32 KiB): half super-block hb's bytes of every tile row -- the dword windows
//    holding ql[64h .. +64) (17 dwords), qh[32h .. +32) (9), sc[8h .. +8) (3) and d (1), h = hb % 2,
//    plus 2 padding dwords: 128 bytes a row, copied by coalesced dword LDS-DMA (32 lanes a row, two
//    rows an instruction) over the two slices before they are needed;
//  * B stages (2 x 32 KiB): thread t < 256 dequantises row t's slice from its raw row (exact fp32,
//    one rounding to 16 bits), written one slice ahead of the MFMAs that read it;
//  * every 128-byte LDS row keeps its 16-byte chunk c at slot c ^ swz(row), so reads of 8 or 16
//    consecutive rows (one chunk each) hit distinct banks;
//  * one barrier per slice: it publishes X(kb+1) and B(kb+1) and frees the stages slice kb read.
// Measured on MI355X (ffn_down 14336 -> 4096, fp16): 57 / 123 / 397 us at M = 128 / 512 / 2048.  The
// bound is LDS fragment traffic beside the MFMAs: each ds_read_b128 of a wave costs its SIMD about
// 12 ns whatever the other wave does, and a 64 x 64 wave tile reads four fragments per four MFMAs.
#include "qvx_deq.hpp"

namespace qvx {

namespace gemmd {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
#define QVX_LDS __attribute__((address_space(3)))

enum { VAR_BF16 = 0, VAR_F16 = 2 };
constexpr uint32_t kRsrcWord3 = 0x00020000u;  // raw buffer, 32-bit data (gfx9)
constexpr int kBM = 128;                      // tokens per tile
constexpr int kBN = 256;                      // weight rows per tile
constexpr int kXStage = kBM * 128;            // one X stage: 128 tokens x 64 16-bit values
constexpr int kBStage = kBN * 128;            // one B stage: 256 rows x 64 16-bit values
constexpr int kRStage = kBN * 128;            // one raw stage: 256 rows x 32 dwords
constexpr int kWaves = 8;                     // two per SIMD
constexpr int kXCopies = kBM * 128 / 1024 / kWaves;   // X copies (1 KiB) per wave per slice (2)
constexpr int kRawCopies = kBN * 32 / 64 / kWaves;    // raw dword copies per wave per half super-block (16)
constexpr int kRawRows = kBN / kWaves;                // tile rows whose raw bytes a wave copies (32)

struct Geo {
  int M, N, K;
  uint32_t row_bytes;
  uint32_t w_records;  // bytes of W the copies may read (the tensor, rounded up to a dword)
  int per_split;       // K slices per workgroup along grid z (even: ranges start a half super-block)
  float* part;         // K-split launches: partial tiles [tile][split][kBM * kBN]
  uint32_t* cnt;       // ... and one arrival counter per tile, zero before the launch
};

template <int N>
__device__ inline void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// LDS through inline asm: the compiler cannot tell these accesses from the stages the in-flight
// buffer_load ... lds copies write and would otherwise wait for every copy (vmcnt(0)) before each of
// them.  The copies are synchronised explicitly (wait_vm before the barrier); lds_wait takes the read
// results as operands, so no use moves above it.
__device__ inline u32x4 lds_read16(uint32_t addr) {
  u32x4 r;
  asm volatile("ds_read_b128 %0, %1" : "=v"(r) : "v"(addr) : "memory");
  return r;
}
__device__ inline void lds_write16(uint32_t addr, u32x4 v) {
  asm volatile("ds_write_b128 %0, %1" ::"v"(addr), "v"(v) : "memory");
}
template <int N>
__device__ inline void lds_wait(u32x4 (&r)[N]) {
  static_assert(N == 4 || N == 6 || N == 8, "lds_wait arity");
  if constexpr (N == 4)
    asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(r[0]), "+v"(r[1]), "+v"(r[2]), "+v"(r[3])::"memory");
  else if constexpr (N == 6)
    asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(r[0]), "+v"(r[1]), "+v"(r[2]), "+v"(r[3]), "+v"(r[4]), "+v"(r[5])::"memory");
  else
    asm volatile("s_waitcnt lgkmcnt(0)"
                 : "+v"(r[0]), "+v"(r[1]), "+v"(r[2]), "+v"(r[3]), "+v"(r[4]), "+v"(r[5]), "+v"(r[6]), "+v"(r[7])::"memory");
}

// Copies global -> LDS (16 or 4 bytes a lane).  Device functions of their own: called straight from
// a lambda in the kernel, the target builtin makes the host pass drop the kernel's launch stub
// without a diagnostic.
__device__ inline void copy_lds16(__amdgpu_buffer_rsrc_t r, QVX_LDS uint8_t* dst, uint32_t voff, uint32_t soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, dst, 16, voff, soff, 0, 0);
}
__device__ inline void copy_lds4(__amdgpu_buffer_rsrc_t r, QVX_LDS uint8_t* dst, uint32_t voff, uint32_t soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, dst, 4, voff, soff, 0, 0);
}

// 16-byte chunk c of row r sits at slot c ^ swz(r) (X and B rows); raw rows use slot c ^ (r % 8).
__device__ inline uint32_t swz(uint32_t r) { return (r ^ ((r >> 3) & 3u)) & 7u; }

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

template <int VAR>
__device__ inline f32x16_t mfma32(const u32x4& a, const u32x4& b, f32x16_t c) {
  if constexpr (VAR == VAR_BF16)
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b), c,
                                                   0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a), __builtin_bit_cast(f16x8_t, b), c, 0,
                                                  0, 0);
}

// Raw row layout (32 dwords): logical dword j of a half super-block window, A = the block's start
// address and A4 = A rounded down to a dword (A - A4 = s is 0 or 2: the 210-byte blocks of a 4-byte
// aligned tensor):
//   j  0..16  A4 + 64h + 4j             ql[64h .. +64) at byte s
//   j 17..25  A4 + 128 + 32h + 4(j-17)  qh[32h .. +32) at byte s
//   j 26..28  A4 + 192 + 8h + 4(j-26)   sc[8h .. +8) at byte s
//   j 29..31  A4 + 208                  d at byte s (29; 30, 31 repeat it)
// Every dword read holds at least one byte of the block, so no read leaves the pages the tensor
// occupies.  Offset of dword j from A4, as base + h * step, packed base | step << 16.
__device__ inline uint32_t raw_piece(uint32_t j) {
  if (j < 17) return (4u * j) | (64u << 16);
  if (j < 26) return (128u + 4u * (j - 17u)) | (32u << 16);
  if (j < 29) return (192u + 4u * (j - 26u)) | (8u << 16);
  return 208u;
}

// Dequantisation of slice e (0, 1) of half super-block h from a raw row (8 chunks, logical order),
// s = the block's byte offset in its dword: element L < 32 of the slice is nibble e of ql[64h + L] |
// bits (4e, 4e+1) of qh[32h + L] << 4 with scale sc[8h + 4e + L/16]; element 32 + L is nibble e of
// ql[64h + 32 + L] | bits (4e+2, 4e+3) of qh[32h + L] << 4 with scale sc[8h + 4e + 2 + L/16]; value
// d * sc * (code - 32).  Step t (0..3) makes elements 16t .. 16t + 15, one scale:
// sc[8h + 4e + t].  Each value is fma(code, d sc, -32 d sc): d sc is exact (11 x 8 bits) and so is
// (code - 32) d sc (<= 24 bits), so the fma returns it exactly, as the reference's float products
// do (a zero product comes out +0 where the reference may give -0).
struct Q6Row {
  uint32_t w[32];
  float sc[4], nsc[4];  // d * sc[8h + 4e + t], -32 d * sc[...]
  uint32_t s;
};

template <int E>
__device__ inline void q6k_prepare(const u32x4 (&rw)[8], uint32_t s, Q6Row& q) {
#pragma unroll
  for (int c = 0; c < 8; ++c) {
    q.w[4 * c] = rw[c].x;
    q.w[4 * c + 1] = rw[c].y;
    q.w[4 * c + 2] = rw[c].z;
    q.w[4 * c + 3] = rw[c].w;
  }
  q.s = s;
  const uint32_t scw = E ? align_bytes(q.w[28], q.w[27], s) : align_bytes(q.w[27], q.w[26], s);
  // d by the hardware conversion (exact for every finite fp16; a NaN d stays NaN)
  const float d = (float)__builtin_bit_cast(_Float16, (uint16_t)((q.w[29] >> (8u * s)) & 0xFFFFu));
  // the signed sub-scales through their unsigned bytes (exact; v_cvt_f32_ubyte<k>)
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const float sb = (float)((scw >> (8u * (uint32_t)k)) & 0xFFu);
    q.sc[k] = d * (sb >= 128.0f ? sb - 256.0f : sb);
    q.nsc[k] = -32.0f * q.sc[k];
  }
}

// Step t: put(c, v8) for chunks c = 2t, 2t + 1 (elements 8c .. 8c + 7).
template <int E, int T, class Put>
__device__ inline void q6k_step(const Q6Row& q, Put&& put) {
  constexpr int half = T >> 1;  // elements 32 half + L, L = 16 (T % 2) .. + 15
  constexpr int hs = 4 * E + 2 * half;  // qh bit pair of this quarter
  float v[16];
#pragma unroll
  for (int jj = 0; jj < 4; ++jj) {
    const int j = 4 * (T & 1) + jj;  // elements L = 4j .. 4j + 3
    const uint32_t ql = align_bytes(q.w[8 * half + j + 1], q.w[8 * half + j], q.s);
    const uint32_t qh = align_bytes(q.w[17 + j + 1], q.w[17 + j], q.s);
    uint32_t hi;
    if constexpr (hs < 4)
      hi = (qh << (4 - hs)) & 0x30303030u;
    else
      hi = (qh >> (hs - 4)) & 0x30303030u;
    const uint32_t code = ((E ? ql >> 4 : ql) & 0x0F0F0F0Fu) | hi;
#pragma unroll
    for (int b = 0; b < 4; ++b)  // (float) of a byte: v_cvt_f32_ubyte<b>
      v[4 * jj + b] = __builtin_fmaf((float)((code >> (8 * b)) & 0xFFu), q.sc[T], q.nsc[T]);
  }
  put(2 * T, reinterpret_cast<const float(&)[8]>(v[0]));
  put(2 * T + 1, reinterpret_cast<const float(&)[8]>(v[8]));
}

}  // namespace gemmd

using namespace gemmd;

template <int P>
using Par = std::integral_constant<int, P>;

template <int VAR>
__global__ __launch_bounds__(512) void k_qgemm_q6k(const uint8_t* __restrict__ W, const uint16_t* __restrict__ X,
                                                   float* __restrict__ Y, Geo geo) {
  constexpr int TM = 2, TN = 2;  // 32 x 32 MFMA tiles per wave: 64 tokens x 64 rows
  constexpr int NF = TM + TN;    // fragments per MFMA step
  __shared__ __attribute__((aligned(1024))) uint8_t xs[2 * kXStage];
  __shared__ __attribute__((aligned(1024))) uint8_t bs[2 * kBStage];
  __shared__ __attribute__((aligned(1024))) uint8_t rs[2 * kRStage];

  const int M = geo.M, N = geo.N, K = geo.K;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave & 1, wn = wave >> 1;
  const bool dq = wave < 4;  // waves 0-3 dequantise (thread t: tile row t), 4-7 only multiply
  const int ln = lane & 31, g = lane >> 5;
  const int n0 = blockIdx.x * kBN, m0 = blockIdx.y * kBM;
  const int nsl = K / 64;
  const int kb0 = blockIdx.z * geo.per_split;
  const int kb1 = min(nsl, kb0 + geo.per_split);
  if (kb0 >= kb1) return;
  const int kl = kb1 - 1;

  QVX_LDS uint8_t* xs_l = (QVX_LDS uint8_t*)xs;
  QVX_LDS uint8_t* rs_l = (QVX_LDS uint8_t*)rs;
  const uint32_t xs_base = (uint32_t)(uintptr_t)xs_l;
  const uint32_t bs_base = (uint32_t)(uintptr_t)(QVX_LDS uint8_t*)bs;
  const uint32_t rs_base = (uint32_t)(uintptr_t)rs_l;

  // X slice kb -> stage p: wave w copies tile rows 8 (w kXCopies + i) .. + 7 (64 lanes x 16 bytes);
  // rows past M read as zeros (buffer range)
  const uint32_t xrow_bytes = (uint32_t)K * 2u;
  const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(X + (size_t)m0 * K), (short)0, (int)((uint32_t)min(kBM, M - m0) * xrow_bytes), (int)kRsrcWord3);
  uint32_t xoff[kXCopies];
#pragma unroll
  for (int i = 0; i < kXCopies; ++i) {
    const uint32_t q = (uint32_t)((wave * kXCopies + i) * 64 + lane), r = q >> 3, p = q & 7u;
    xoff[i] = r * xrow_bytes + 16u * (p ^ swz(r));
  }
  auto issue_x = [&](int kb, int p) {
    QVX_LDS uint8_t* dst = xs_l + p * kXStage + wave * kXCopies * 1024;
#pragma unroll
    for (int i = 0; i < kXCopies; ++i) copy_lds16(xr, dst + i * 1024, xoff[i], (uint32_t)kb * 128u);
  };

  // Raw copies of half super-block hb: wave w fills tile rows 32w .. 32w + 31, instruction i rows
  // R = 32w + 2i + g (g = lane / 32), lane position q = lane % 32 of the row's 128 LDS bytes holding
  // logical dword 4 ((q / 4) ^ (R % 8)) + q % 4.  R % 8 = (g + 2i) % 8 takes four values (i % 4),
  // each with its own dword pattern; rows 2i apart differ by 2i row_bytes, a multiple of 4 (the
  // buffer's scalar offset).  Rows past N read as zeros (buffer range) or hold bytes of the last
  // row's dword; their columns are dropped.
  const __amdgpu_buffer_rsrc_t wr =
      __builtin_amdgcn_make_buffer_rsrc((void*)W, (short)0, (int)geo.w_records, (int)kRsrcWord3);
  const uint32_t row0_off = (uint32_t)(n0 + kRawRows * wave + g) * geo.row_bytes;
  uint32_t piece[4];
#pragma unroll
  for (int pq = 0; pq < 4; ++pq) {
    const uint32_t q = (uint32_t)ln, rsw = (uint32_t)(g + 2 * pq) & 7u;
    piece[pq] = raw_piece(4u * ((q >> 2) ^ rsw) + (q & 3u));
  }
  // copies half (0: i = 0..7, 1: i = 8..15) of half super-block hb into raw stage st
  auto issue_raw = [&](int hb, int st, int half) {
    const uint32_t u = (uint32_t)hb >> 1, h = (uint32_t)hb & 1u;
    const uint32_t a4 = (row0_off + 210u * u) & ~3u;
    uint32_t voff[4];
#pragma unroll
    for (int pq = 0; pq < 4; ++pq) voff[pq] = a4 + (piece[pq] & 0xFFFFu) + h * (piece[pq] >> 16);
    QVX_LDS uint8_t* dst = rs_l + st * kRStage + wave * kRawCopies * 256;
#pragma unroll
    for (int ii = 0; ii < kRawCopies / 2; ++ii) {
      const int i = half * (kRawCopies / 2) + ii;
      copy_lds4(wr, dst + i * 256, voff[i & 3], (uint32_t)(2 * i) * geo.row_bytes);
    }
  };

  // Thread t < 256 dequantises tile row t: its raw row at rs + st * kRStage + 128 t (chunk c at slot
  // c ^ (t % 8)); s = the row's block offset in its dword for super-block u: (row offset + 2u) % 4.
  const uint32_t rrow = rs_base + (uint32_t)tid * 128u, rsw_t = (uint32_t)tid & 7u;
  const uint32_t s_row = ((uint32_t)(n0 + tid) * geo.row_bytes) & 3u;
  const uint32_t bw_row = bs_base + (uint32_t)tid * 128u, bw_swz = swz((uint32_t)tid);
  auto read_raw = [&](int st, u32x4 (&rw)[8]) {
#pragma unroll
    for (int c = 0; c < 8; ++c) rw[c] = lds_read16(rrow + (uint32_t)st * kRStage + 16u * ((uint32_t)c ^ rsw_t));
  };
  // B chunk c of this thread's row into B stage p
  auto b_put = [&](uint32_t row, int c, const float (&v)[8]) {
    const u32x4 w = {pack2<VAR>(v[0], v[1]), pack2<VAR>(v[2], v[3]), pack2<VAR>(v[4], v[5]), pack2<VAR>(v[6], v[7])};
    lds_write16(row + 16u * ((uint32_t)c ^ bw_swz), w);
  };
  auto row_s = [&](int kb) { return (s_row + 2u * ((uint32_t)kb >> 2)) & 3u; };

  // fragment reads of step t: A row 64 wm + 32 i + ln, B row 64 wn + 32 j + ln, chunk 2t + g
  const uint32_t sw = swz((uint32_t)ln);
  uint32_t a_rel[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) a_rel[t] = (uint32_t)(32 * TM * wm + ln) * 128u + 16u * ((2u * (uint32_t)t + (uint32_t)g) ^ sw);
  const uint32_t b_row0 = (uint32_t)(32 * TN * wn + ln) * 128u;
  auto read_step = [&](int p, int t, u32x4 (&f)[NF]) {
    const uint32_t xa = xs_base + (uint32_t)p * kXStage + a_rel[t];
    const uint32_t ba = bs_base + (uint32_t)p * kBStage + b_row0 + (a_rel[t] & 127u);
#pragma unroll
    for (int i = 0; i < TM; ++i) f[i] = lds_read16(xa + 4096u * (uint32_t)i);
#pragma unroll
    for (int j = 0; j < TN; ++j) f[TM + j] = lds_read16(ba + 4096u * (uint32_t)j);
  };

  f32x16_t acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

  // Slices are counted from kb0 (even, so the range starts a half super-block): slice r = kb - kb0
  // reads X / B stage r % 2, and half super-block m = r / 2 lives in raw stage m % 2.  Raw(m) is
  // copied during slices 2m - 3 (first half) and 2m - 2 (second half), after the barrier that ended
  // the last read of raw(m - 2), and has landed by the end of slice 2m - 2: slice 2m - 1 dequantises
  // slice 2m from it.  Copies past the range are skipped (uniform branch; the wait below adapts).
  const int hb0 = kb0 >> 1, mlast = (kl - kb0) >> 1;
  // Prologue: X(kb0), raw(0) landed, B(kb0) written; raw(1)'s first half in flight.
  issue_x(kb0, 0);
  issue_raw(hb0, 0, 0);
  issue_raw(hb0, 0, 1);
  if (mlast >= 1) {
    issue_raw(hb0 + 1, 1, 0);
    wait_vm<kRawCopies / 2>();
  } else {
    wait_vm<0>();
  }
  __builtin_amdgcn_s_barrier();  // raw(0) rows come from every wave's copies
  if (dq) {
    u32x4 rw[8];
    read_raw(0, rw);
    lds_wait<8>(rw);
    Q6Row q;
    q6k_prepare<0>(rw, row_s(kb0), q);
    auto put = [&](int c, const float (&v)[8]) { b_put(bw_row, c, v); };
    q6k_step<0, 0>(q, put);
    q6k_step<0, 1>(q, put);
    q6k_step<0, 2>(q, put);
    q6k_step<0, 3>(q, put);
  }
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
  __builtin_amdgcn_s_barrier();

  auto slice = [&](int kb, auto par) {
    constexpr int p = decltype(par)::value;  // (kb - kb0) % 2
    const int r = kb - kb0;
    // X(kb+1) into stage 1-p (read by slice kb-1, freed by the last barrier); then raw copies:
    // odd r: first half of raw((r + 3) / 2); even r: second half of raw((r + 2) / 2)
    issue_x(min(kb + 1, kl), 1 - p);
    const int m = p ? (r + 3) >> 1 : (r + 2) >> 1;
    const bool raw = m <= mlast;
    if (raw) issue_raw(hb0 + m, m & 1, p ? 0 : 1);
    // raw row of slice kb+1 (half super-block (r + 1) / 2) for this thread's dequantisation; its
    // parity E is 1 - p (kb0 is even; the last slice dequantises a copy of itself into a stage
    // nothing reads again)
    constexpr int E = 1 - p;
    u32x4 rw[8];
    if (dq) read_raw(((r + 1) >> 1) & 1, rw);
    u32x4 f[2][NF];
    read_step(p, 0, f[0]);
    Q6Row q;
    if (dq) {
      lds_wait<8>(rw);
      q6k_prepare<E>(rw, row_s(min(kb + 1, kl)), q);
    }
    const uint32_t brow = bw_row + (uint32_t)(1 - p) * kBStage;
    auto put = [&](int c, const float (&v)[8]) { b_put(brow, c, v); };
    // step t: MFMAs of slice kb's K columns 16t .. 16t + 15 (fragments of step t+1 read meanwhile)
    // beside dequantisation step t of slice kb+1 into B stage 1-p
    auto step = [&](auto tt) {
      constexpr int t = decltype(tt)::value;
      lds_wait<NF>(f[t & 1]);
      if constexpr (t + 1 < 4) read_step(p, t + 1, f[(t + 1) & 1]);
      // keep the reads ahead of this step's MFMAs and dequantisation (the scheduler does not know
      // their latency and would sink them to the next wait)
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = mfma32<VAR>(f[t & 1][i], f[t & 1][TM + j], acc[i][j]);
      if (dq) q6k_step<E, t>(q, put);
    };
    step(Par<0>{});
    step(Par<1>{});
    step(Par<2>{});
    step(Par<3>{});
    // X(kb+1) landed; odd r: the raw copies just issued may fly, even r: they complete raw(m).
    // Then this wave's LDS writes; the barrier publishes slice kb+1 and frees stage p.
    if (p && raw)
      wait_vm<kRawCopies / 2>();
    else
      wait_vm<0>();
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
    __builtin_amdgcn_s_barrier();
  };
  int kb = kb0;
  for (; kb + 1 < kb1; kb += 2) {  // the back edge always follows an odd slice
    slice(kb, Par<0>{});
    slice(kb + 1, Par<1>{});
  }
  if (kb < kb1) slice(kb, Par<0>{});

  // K split: the split that finishes a tile last sums the partials in split order and stores it.
  if (gridDim.z > 1) {
    constexpr int NA = TM * TN * 16;
    const int t = (int)(blockIdx.y * gridDim.x + blockIdx.x);
    wait_vm<0>();  // no LDS copy in flight when the flag word of xs is written
    float v[NA];
#pragma unroll
    for (int a = 0; a < NA; ++a) v[a] = acc[a / (TN * 16)][(a / 16) % TN][a % 16];
    if (!split_k_last<NA, 512>(v, geo.part + (size_t)t * gridDim.z * (NA * 512), geo.cnt + t, (int)gridDim.z,
                               (int)blockIdx.z, tid, reinterpret_cast<int*>(xs)))
      return;
#pragma unroll
    for (int a = 0; a < NA; ++a) acc[a / (TN * 16)][(a / 16) % TN][a % 16] = v[a];
  }

  // C layout of v_mfma_f32_32x32x*: element e of lane l is row 8*(e/4) + 4*(l/32) + e%4, col l%32.
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int n = n0 + 32 * TN * wn + 32 * j + ln;
      if (n >= N) continue;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int m = m0 + 32 * (TM * wm + i) + 8 * (e >> 2) + 4 * g + (e & 3);
        if (m < M) Y[(size_t)m * N + n] = acc[i][j][e];
      }
    }
}

namespace {

// 128-token tiles; K split (partial tiles summed in split order by the last split of each tile)
// while the grid is smaller than ~one workgroup per CU and each range keeps >= 8 slices.  Ranges are
// an even number of slices, none empty.
inline void q6k_plan(int M, int N, int K, int& splits, int& per) {
  const int tiles = ((N + kBN - 1) / kBN) * ((M + kBM - 1) / kBM), nsl = K / 64;
  splits = 1;
  while (tiles * splits < 200 && nsl / (splits * 2) >= 8) splits *= 2;
  per = (nsl + splits - 1) / splits;
  per += per & 1;
  splits = (nsl + per - 1) / per;
}

inline int q6k_tiles(int M, int N) { return ((N + kBN - 1) / kBN) * ((M + kBM - 1) / kBM); }

template <int VAR>
bool launch_var(float* out, const void* w, const uint16_t* X, int M, int N, int K, size_t row_bytes, void* split_ws,
                hipStream_t s) {
  static LdsLimit lim;
  if (!lds_ready(reinterpret_cast<const void*>(&k_qgemm_q6k<VAR>), lim, 0)) return false;
  int splits, per;
  q6k_plan(M, N, K, splits, per);
  if (splits > 1 && !split_ws) return false;
  const uint32_t wrec = (uint32_t)(((size_t)N * row_bytes + 3u) & ~(size_t)3u);
  const size_t pbytes = (size_t)q6k_tiles(M, N) * splits * kBM * kBN * 4;
  float* part = splits > 1 ? static_cast<float*>(split_ws) : nullptr;
  uint32_t* cnt = splits > 1 ? reinterpret_cast<uint32_t*>(static_cast<uint8_t*>(split_ws) + pbytes) : nullptr;
  Geo geo{M, N, K, (uint32_t)row_bytes, wrec, per, part, cnt};
  dim3 grid((N + kBN - 1) / kBN, (M + kBM - 1) / kBM, splits);
  k_qgemm_q6k<VAR><<<grid, 64 * kWaves, 0, s>>>(static_cast<const uint8_t*>(w), X, out, geo);
  return true;
}

}  // namespace

// 1 if the dequantising MFMA GEMM takes this call: a Q6_K weight (K whole super-blocks), X 16-byte
// and W 4-byte aligned (dword windows, block offsets 0 or 2), one tile's X rows and the whole weight
// within 31-bit buffer offsets.
bool qgemm_deq_supported(uint32_t t, const void* w, const uint16_t* X, int K, int N, size_t row_bytes) {
  if (t != T_Q6_K || K <= 0 || K % 256 != 0 || N <= 0) return false;
  if ((reinterpret_cast<uintptr_t>(X) & 15u) || (reinterpret_cast<uintptr_t>(w) & 3u)) return false;
  if ((size_t)kBM * (size_t)K * 2u >= (1u << 31)) return false;
  if ((size_t)N * row_bytes + 3u >= (1u << 31)) return false;
  return true;
}

// Workspace of the launch's K split: the partial tiles, then the tile counters (256-byte aligned;
// the counters are the last `counters` bytes and must be zero at the launch), or 0 without a split.
size_t qgemm_deq_split_bytes(int M, int N, int K, size_t* counters) {
  int splits, per;
  q6k_plan(M, N, K, splits, per);
  if (splits <= 1) return *counters = 0;
  const size_t tiles = (size_t)q6k_tiles(M, N);
  *counters = (tiles * 4 + 255) & ~(size_t)255;
  return tiles * splits * kBM * kBN * 4 + *counters;
}

// Launches the GEMM (X already 16-bit: fp16 for the fp16 variant, bf16 for the bf16 one); split_ws:
// the qgemm_deq_split_bytes workspace, counters zero.
bool launch_qgemm_deq(uint32_t t, float* out, const void* w, const uint16_t* X, int M, int N, int K, size_t row_bytes,
                      bool bf16, void* split_ws, hipStream_t s) {
  if (t != T_Q6_K) return false;
  return bf16 ? launch_var<VAR_BF16>(out, w, X, M, N, K, row_bytes, split_ws, s)
              : launch_var<VAR_F16>(out, w, X, M, N, K, row_bytes, split_ws, s);
}

}  // namespace qvx
