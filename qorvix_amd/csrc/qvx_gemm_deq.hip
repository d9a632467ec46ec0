// qvx_gemm_deq.hip -- prefill GEMM of Q6_K weights (Q4_K has its own kernels in qvx_gemm.hip): the
// weight rows of each K slice are dequantised in registers into a 16-bit B tile in LDS, then bf16 /
// fp16 MFMA.
//
// out[m, r] = sum_k X[m, k] * dequant(W)[r, k],  X [M, K] 16-bit, W raw GGUF blocks [N rows, K],
// out fp32 [M, N].  No reference counterpart (the reference prefills token by token); the semantics
// are qmatmulN's (runtime/src/qmatmul.cpp:64-115) with X converted fp16 -> fp32 exactly.  Each
// weight element is the reference's exact dequantised value (runtime/src/dequant.cpp:38-210) rounded
// once to bf16 / fp16.
//
// Workgroup = 256 threads (4 waves, one per SIMD) computing a BM x 256 tile (BM = 256 or 128 tokens x
// 256 weight rows); wave w owns tokens (w / 2) BM/2 .. + BM/2 - 1 and weight rows 128 (w % 2) .. +127:
// BM/64 x 4 tiles of v_mfma_f32_32x32x16_{bf16,f16} (acc in registers).  K advances in slices of 64:
//  * X slice (BM rows x 128 bytes) is copied global -> LDS by buffer_load ... lds, two stages;
//  * thread t dequantises weight row t of the tile for the slice: its raw bytes come from global
//    memory into registers two slices ahead (Q6_K: one row's 64 elements need 29 dwords), the 64
//    values are computed exactly in fp32, rounded once to 16 bits and written to the B stage as 8
//    chunks of 16 bytes;
//  * both tiles are 128-byte rows whose 16-byte chunk c sits at slot c ^ swz(row), so the fragment
//    reads of 16 consecutive rows (one chunk each) hit distinct banks;
//  * one barrier per slice: it publishes X(kb+1) and B(kb+1) (written during slice kb) and frees the
//    stages slice kb read.
#include "qvx_deq.hpp"

namespace qvx {

namespace gemmd {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef int i32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4a4_t __attribute__((ext_vector_type(4), aligned(4)));  // dword-aligned 16 bytes
typedef uint32_t u32x2a4_t __attribute__((ext_vector_type(2), aligned(4)));  // dword-aligned 8 bytes
#define QVX_LDS __attribute__((address_space(3)))

enum { VAR_BF16 = 0, VAR_F16 = 2 };
constexpr uint32_t kRsrcWord3 = 0x00020000u;  // raw buffer, 32-bit data (gfx9)
constexpr int kBN = 256;                      // weight rows per tile
constexpr int kBStage = kBN * 128;            // one B stage: 256 rows x 64 16-bit values

struct Geo {
  int M, N, K;
  uint32_t row_bytes;
  int per_split;   // K slices per workgroup along grid z
  int atomic_out;  // 1: accumulate into a zeroed output (split K)
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
  static_assert(N == 6 || N == 8, "lds_wait arity");
  if constexpr (N == 6)
    asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(r[0]), "+v"(r[1]), "+v"(r[2]), "+v"(r[3]), "+v"(r[4]), "+v"(r[5])::"memory");
  else
    asm volatile("s_waitcnt lgkmcnt(0)"
                 : "+v"(r[0]), "+v"(r[1]), "+v"(r[2]), "+v"(r[3]), "+v"(r[4]), "+v"(r[5]), "+v"(r[6]), "+v"(r[7])::"memory");
}

// One 16-byte-per-lane copy global -> LDS.  A device function of its own: called straight from a
// lambda in the kernel, the target builtin would make the host pass drop the kernel's launch stub
// without a diagnostic.
__device__ inline void copy_lds16(__amdgpu_buffer_rsrc_t r, QVX_LDS uint8_t* dst, uint32_t voff, uint32_t soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, dst, 16, voff, soff, 0, 0);
}

// 16-byte chunk c of row r sits at slot c ^ swz(r).
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

// ---- weight slices ------------------------------------------------------------------------------
// Slice<T>: one weight row's 64 values of K slice kb.  load() issues the row's raw reads for the
// slice (global -> registers, ahead of use); emit() turns them into values and hands them to put(c,
// v8) as 8 chunks of 8 (elements 8c .. 8c + 7).  kLoads = a lower bound on the vector memory
// instructions load() issues (the pipeline's vmcnt wait counts them).

template <uint32_t T>
struct Slice;

// Q6_K: slice kb = elements 64 q4 .. 64 q4 + 63 (q4 = kb % 4) of super-block u = kb / 4, i.e. half
// h = q4 / 2, nibble / bit-pair set e = q4 % 2.  Element L < 32: code = nibble e of ql[64h + L] |
// bits (4e, 4e+1) of qh[32h + L] << 4, scale sc[8h + 4e + L/16]; element 32 + L: nibble e of
// ql[64h + 32 + L] | bits (4e+2, 4e+3) of qh[32h + L] << 4, scale sc[8h + 4e + 2 + L/16]; value
// d * sc * (code - 32), exact in fp32 (<= 23 significant bits).
// The 210-byte blocks of a 4-byte aligned tensor start at byte offsets s = 0 or 2 of a dword, and
// ql, qh, sc and d sit at multiples of 4 from the block start: each piece is read as the dword-aligned
// window holding it (17, 9, 2 and 1 dwords) and shifted by s in registers.  Every dword read holds
// at least one byte of the block, so no read leaves the pages the tensor occupies.
__device__ inline uint32_t ldg4(const uint8_t* p) { return *reinterpret_cast<const uint32_t*>(p); }
__device__ inline u32x2a4_t ldg8a4(const uint8_t* p) { return *reinterpret_cast<const u32x2a4_t*>(p); }
__device__ inline u32x4a4_t ldg16a4(const uint8_t* p) { return *reinterpret_cast<const u32x4a4_t*>(p); }

template <>
struct Slice<T_Q6_K> {
  static constexpr int kLoads = 10;  // 4 + 1 (ql), 2 + 1 (qh), 1 (sc), 1 (d)
  struct Raw {
    u32x4a4_t l[4], h[2];
    u32x2a4_t sc;
    uint32_t le, he, dd;
  };
  __device__ static const uint8_t* block(const uint8_t* row, int kb) { return row + 210u * ((uint32_t)kb >> 2); }
  __device__ static void load(const uint8_t* row, int kb, Raw& r) {
    const uint32_t h = ((uint32_t)kb >> 1) & 1u, e = (uint32_t)kb & 1u;
    const uint8_t* a = block(row, kb);
    const uint8_t* a4 = a - (reinterpret_cast<uintptr_t>(a) & 3u);  // dword holding the block's byte 0
    const uint8_t* pl = a4 + 64u * h;
    const uint8_t* ph = a4 + 128u + 32u * h;
    r.l[0] = ldg16a4(pl);
    r.l[1] = ldg16a4(pl + 16);
    r.l[2] = ldg16a4(pl + 32);
    r.l[3] = ldg16a4(pl + 48);
    r.le = ldg4(pl + 64);
    r.h[0] = ldg16a4(ph);
    r.h[1] = ldg16a4(ph + 16);
    r.he = ldg4(ph + 32);
    r.sc = ldg8a4(a4 + 192u + 8u * h + 4u * e);
    r.dd = ldg4(a4 + 208u);
  }
  template <class Put>
  __device__ static void emit(const uint8_t* row, const Raw& r, int kb, Put&& put) {
    const uint32_t e = (uint32_t)kb & 1u;
    const uint32_t s = (uint32_t)(reinterpret_cast<uintptr_t>(block(row, kb)) & 3u);
    const uint32_t lw[17] = {r.l[0].x, r.l[0].y, r.l[0].z, r.l[0].w, r.l[1].x, r.l[1].y, r.l[1].z, r.l[1].w,
                             r.l[2].x, r.l[2].y, r.l[2].z, r.l[2].w, r.l[3].x, r.l[3].y, r.l[3].z, r.l[3].w, r.le};
    const uint32_t hw[9] = {r.h[0].x, r.h[0].y, r.h[0].z, r.h[0].w, r.h[1].x, r.h[1].y, r.h[1].z, r.h[1].w, r.he};
    const uint32_t scw = align_bytes(r.sc.y, r.sc.x, s);  // sc[8h + 4e .. +3] as 4 signed bytes
    const float d = f16_bits_to_f32((r.dd >> (8u * s)) & 0xFFFFu);  // s is 0 or 2: d never straddles
    // the signed sub-scales through their unsigned bytes (exact): hipcc for gfx950 folds a
    // sign-extended byte converted to float into v_cvt_f32_u32 with an SDWA sext source, which turns
    // every negative scale into ~4.3e9
    float ds[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const float sb = (float)((scw >> (8u * (uint32_t)k)) & 0xFFu);
      ds[k] = d * (sb >= 128.0f ? sb - 256.0f : sb);
    }
#pragma unroll
    for (int c = 0; c < 8; ++c) {  // elements 8c .. 8c + 7 = 32 half + L, L = 8 (c % 4) ..
      const int half = c >> 2;
      float v8[8];
#pragma unroll
      for (int jj = 0; jj < 2; ++jj) {
        const int j = 2 * (c & 3) + jj;  // 4 elements L = 4j .. 4j + 3
        const uint32_t ql = align_bytes(lw[8 * half + j + 1], lw[8 * half + j], s);
        const uint32_t qh = align_bytes(hw[j + 1], hw[j], s);
        const uint32_t code = ((ql >> (4u * e)) & 0x0F0F0F0Fu) | (((qh >> (4u * e + 2u * half)) & 0x03030303u) << 4);
#pragma unroll
        for (int b = 0; b < 4; ++b) {
          const int L = 4 * j + b;
          v8[4 * jj + b] = ds[2 * half + (L >> 4)] * (float)((int)((code >> (8 * b)) & 0xFFu) - 32);
        }
      }
      put(c, v8);
    }
  }
};

}  // namespace gemmd

using namespace gemmd;

template <int P>
using Par = std::integral_constant<int, P>;

template <uint32_t T, int VAR, int BM>
__global__ __launch_bounds__(256) void k_qgemm_deq(const uint8_t* W, const uint16_t* __restrict__ X,
                                                   float* __restrict__ Y, Geo geo) {
  using S = Slice<T>;
  constexpr int TM = BM / 64;        // 32-token tiles per wave
  constexpr int XI = BM / 32;        // X copies (1 KB) per wave per slice
  constexpr int XSTAGE = BM * 128;   // bytes of one X slice
  constexpr int NL = S::kLoads;
  __shared__ __attribute__((aligned(1024))) uint8_t xs[2 * XSTAGE];
  __shared__ __attribute__((aligned(1024))) uint8_t bs[2 * kBStage];

  const int M = geo.M, N = geo.N, K = geo.K;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  const int ln = lane & 31, g = lane >> 5;
  const int n0 = blockIdx.x * kBN, m0 = blockIdx.y * BM;
  const int nsl = K / 64;
  const int kb0 = blockIdx.z * geo.per_split;
  const int kb1 = min(nsl, kb0 + geo.per_split);
  if (kb0 >= kb1) return;

  // X slice kb -> stage p: wave w copies tile rows 8 (w XI + i) .. + 7 (64 lanes x 16 bytes each)
  const uint32_t xrow_bytes = (uint32_t)K * 2u;
  const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(X + (size_t)m0 * K), (short)0, (int)((uint32_t)min(BM, M - m0) * xrow_bytes), (int)kRsrcWord3);
  uint32_t xoff[XI];
#pragma unroll
  for (int i = 0; i < XI; ++i) {
    const uint32_t q = (uint32_t)((wave * XI + i) * 64 + lane), r = q >> 3, p = q & 7u;
    xoff[i] = r * xrow_bytes + 16u * (p ^ swz(r));
  }
  QVX_LDS uint8_t* xs_l = (QVX_LDS uint8_t*)xs;
  auto issue_x = [&](int kb, int p) {
    QVX_LDS uint8_t* dst = xs_l + p * XSTAGE + wave * XI * 1024;
#pragma unroll
    for (int i = 0; i < XI; ++i)
      copy_lds16(xr, dst + i * 1024, xoff[i], (uint32_t)kb * 128u);
  };

  // this thread dequantises tile row tid (rows past N repeat the last row; their columns are dropped)
  const uint8_t* wrow = W + (size_t)min(n0 + tid, N - 1) * geo.row_bytes;
  const uint32_t xs_base = (uint32_t)(uintptr_t)xs_l;
  const uint32_t bs_base = (uint32_t)(uintptr_t)(QVX_LDS uint8_t*)bs;
  const uint32_t bw_rel = (uint32_t)tid * 128u, bw_swz = swz((uint32_t)tid);
  auto write_b = [&](const typename S::Raw& raw, int kb, int p) {
    const uint32_t row = bs_base + (uint32_t)p * kBStage + bw_rel;
    S::emit(wrow, raw, kb, [&](int c, const float (&v)[8]) {
      const u32x4 w = {pack2<VAR>(v[0], v[1]), pack2<VAR>(v[2], v[3]), pack2<VAR>(v[4], v[5]), pack2<VAR>(v[6], v[7])};
      lds_write16(row + 16u * ((uint32_t)c ^ bw_swz), w);
    });
  };
  // raw reads of slice kb, ordered after the X copies issued before them (the vmcnt wait below
  // counts on it): the empty asm orders memory operations, and W is not restrict-qualified, so its
  // reads are not treated as invariant and moved across it
  auto load_w = [&](int kb, typename S::Raw& raw) {
    asm volatile("" ::: "memory");
    S::load(wrow, kb, raw);
  };

  // fragment reads of step t: A row 32 (TM wm + i) + ln, B row 128 wn + 32 j + ln, chunk 2t + g
  const uint32_t sw = swz((uint32_t)ln);
  uint32_t a_rel[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) a_rel[t] = (uint32_t)(32 * TM * wm + ln) * 128u + 16u * ((2u * (uint32_t)t + (uint32_t)g) ^ sw);
  const uint32_t b_row0 = (uint32_t)(128 * wn + ln) * 128u;
  constexpr int NF = TM + 4;
  auto read_step = [&](int p, int t, u32x4 (&f)[NF]) {
    const uint32_t xa = xs_base + (uint32_t)p * XSTAGE + a_rel[t];
    const uint32_t ba = bs_base + (uint32_t)p * kBStage + b_row0 + (a_rel[t] & 127u);
#pragma unroll
    for (int i = 0; i < TM; ++i) f[i] = lds_read16(xa + 4096u * (uint32_t)i);
#pragma unroll
    for (int j = 0; j < 4; ++j) f[TM + j] = lds_read16(ba + 4096u * (uint32_t)j);
  };

  f32x16_t acc[TM][4];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

  // Stages and raw registers alternate: slice kb uses stage / raw set (kb - kb0) % 2.  Every slice
  // issues the same copies, reads and dequantisation, clamped to the last slice of the range (the
  // surplus lands in a stage nothing reads again): one shape per iteration, so the compiler's own
  // waits for the raw registers stay exact.
  const int kl = kb1 - 1;
  typename S::Raw raw[2];
  // Prologue: X(kb0) landed and B(kb0) written; raw W(kb0+1) in flight.
  issue_x(kb0, 0);
  load_w(kb0, raw[0]);
  load_w(min(kb0 + 1, kl), raw[1]);
  write_b(raw[0], kb0, 0);
  wait_vm<NL>();
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
  __builtin_amdgcn_s_barrier();

  auto slice = [&](int kb, auto par) {
    constexpr int p = decltype(par)::value;
    // X(kb+1) into stage 1-p (read by slice kb-1, freed by the last barrier), then raw W(kb+2)
    issue_x(min(kb + 1, kl), 1 - p);
    load_w(min(kb + 2, kl), raw[p]);
    // MFMAs of slice kb, the fragments of step t+1 read while step t's run
    u32x4 f[2][NF];
    read_step(p, 0, f[0]);
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      lds_wait<NF>(f[t & 1]);
      if (t + 1 < 4) read_step(p, t + 1, f[(t + 1) & 1]);
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = mfma32<VAR>(f[t & 1][i], f[t & 1][TM + j], acc[i][j]);
    }
    // B(kb+1) into stage 1-p from raw W(kb+1), read during slice kb-1 (the prologue for kb0)
    write_b(raw[1 - p], min(kb + 1, kl), 1 - p);
    // X(kb+1) landed (only the raw W(kb+2) reads, issued after it, may fly) and this wave's LDS
    // writes done; the barrier then publishes slice kb+1 and frees stage p
    wait_vm<NL>();
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
    __builtin_amdgcn_s_barrier();
  };
  int kb = kb0;
  for (; kb + 1 < kb1; kb += 2) {  // the back edge always follows a raw set 1 slice
    slice(kb, Par<0>{});
    slice(kb + 1, Par<1>{});
  }
  if (kb < kb1) slice(kb, Par<0>{});
  wait_vm<0>();  // the surplus raw reads

  // C layout of v_mfma_f32_32x32x*: element e of lane l is row 8*(e/4) + 4*(l/32) + e%4, col l%32.
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int n = n0 + 128 * wn + 32 * j + ln;
      if (n >= N) continue;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int m = m0 + 32 * (TM * wm + i) + 8 * (e >> 2) + 4 * g + (e & 3);
        if (m < M) {
          float* dst = Y + (size_t)m * N + n;
          if (geo.atomic_out)
            unsafeAtomicAdd(dst, acc[i][j][e]);
          else
            *dst = acc[i][j][e];
        }
      }
    }
}

void launch_zero(float* p, size_t n, hipStream_t s);

namespace {

inline int split_per(int nsl, int splits) { return (nsl + splits - 1) / splits; }

template <uint32_t T, int VAR, int BM>
bool launch_bm(float* out, const void* w, const uint16_t* X, int M, int N, int K, size_t row_bytes, int splits,
               bool zeroed, hipStream_t s) {
  static LdsLimit lim;
  if (!lds_ready(reinterpret_cast<const void*>(&k_qgemm_deq<T, VAR, BM>), lim, 0)) return false;
  const int nsl = K / 64;
  const int per = split_per(nsl, splits);
  splits = (nsl + per - 1) / per;
  if (splits > 1 && !zeroed) launch_zero(out, (size_t)M * N, s);
  Geo geo{M, N, K, (uint32_t)row_bytes, per, splits > 1 ? 1 : 0};
  dim3 grid((N + kBN - 1) / kBN, (M + BM - 1) / BM, splits);
  k_qgemm_deq<T, VAR, BM><<<grid, 256, 0, s>>>(static_cast<const uint8_t*>(w), X, out, geo);
  return true;
}

// 256-token tiles when they alone give ~one workgroup per CU; else 128-token tiles, splitting K
// (fp32 atomics into a zeroed output) while the grid is smaller than that.
inline void deq_plan(int M, int N, int K, int& bm, int& splits) {
  const int nt = (N + kBN - 1) / kBN, nsl = K / 64;
  splits = 1;
  if (nt * ((M + 255) / 256) >= 200) {
    bm = 256;
    return;
  }
  bm = 128;
  const int tiles = nt * ((M + 127) / 128);
  while (tiles * splits < 200 && nsl / (splits * 2) >= 8) splits *= 2;
  const int per = split_per(nsl, splits);
  splits = (nsl + per - 1) / per;
}

template <uint32_t T, int VAR>
bool launch_t(float* out, const void* w, const uint16_t* X, int M, int N, int K, size_t row_bytes, bool zeroed,
              hipStream_t s) {
  int bm, splits;
  deq_plan(M, N, K, bm, splits);
  if (bm == 256) return launch_bm<T, VAR, 256>(out, w, X, M, N, K, row_bytes, splits, zeroed, s);
  return launch_bm<T, VAR, 128>(out, w, X, M, N, K, row_bytes, splits, zeroed, s);
}

template <int VAR>
bool launch_var(uint32_t t, float* out, const void* w, const uint16_t* X, int M, int N, int K, size_t row_bytes,
                bool zeroed, hipStream_t s) {
  switch (t) {
    case T_Q6_K: return launch_t<T_Q6_K, VAR>(out, w, X, M, N, K, row_bytes, zeroed, s);
    default: return false;
  }
}

}  // namespace

// 1 if the dequantising MFMA GEMM takes this call: a Q6_K weight (the generic per-element form runs
// every other type correctly but ~8x slower than dequantise-then-library at large M, so it is not
// routed), K a multiple of 64, X 16-byte aligned, the weight 4-byte aligned (Q6_K reads dword
// windows), and one tile's rows within 32-bit buffer offsets.
bool qgemm_deq_supported(uint32_t t, const void* w, const uint16_t* X, int K, size_t row_bytes) {
  if (t != T_Q6_K || K <= 0 || K % 64 != 0) return false;
  if ((reinterpret_cast<uintptr_t>(X) & 15u) || (reinterpret_cast<uintptr_t>(w) & 3u)) return false;
  if ((size_t)256 * (size_t)K * 2u >= (1u << 31)) return false;
  (void)row_bytes;
  return can_dequantize(t);
}

// The tile plan (for callers that zero the output of a K-split launch themselves).
bool qgemm_deq_splits(int M, int N, int K) {
  int bm, splits;
  deq_plan(M, N, K, bm, splits);
  return splits > 1;
}

// Launches the GEMM (X already 16-bit: fp16 for the fp16 variant, bf16 for the bf16 one).
// zeroed: the caller zeroed the output of a K-split launch.
bool launch_qgemm_deq(uint32_t t, float* out, const void* w, const uint16_t* X, int M, int N, int K, size_t row_bytes,
                      bool bf16, bool zeroed, hipStream_t s) {
  return bf16 ? launch_var<VAR_BF16>(t, out, w, X, M, N, K, row_bytes, zeroed, s)
              : launch_var<VAR_F16>(t, out, w, X, M, N, K, row_bytes, zeroed, s);
}

}  // namespace qvx
