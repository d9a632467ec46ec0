// qvx_gemm.hip -- prefill GEMM (M >= 128) over raw GGUF Q4_K blocks on gfx950 matrix cores.
//
// out[m, r] = sum_k X[m, k] * dequant(W)[r, k],  X [M, K] 16-bit, W Q4_K [N rows, K], out fp32 [M, N].
// No reference counterpart (the reference prefills token by token); the semantics are qmatmulN's
// (runtime/src/qmatmul.cpp:64-115) with X converted fp16 -> fp32 exactly.
//
// Workgroup = 512 threads (8 waves, two per SIMD) computing a BM x 256 output tile (BM = 64..256
// tokens x 256 weight rows); wave w owns weight rows 32w..32w+31 of the tile and all BM tokens, so
// every weight element is dequantised once per workgroup, and on each SIMD one wave's
// dequantisation VALU, copy issue and LDS waits run beside the other wave's MFMAs.
// v_mfma_f32_32x32x16_{bf16,f16}.
//
// K advances in slices of 64 elements = one 64-element group c of a Q4_K super-block:
//  * X slice (BM x 64 16-bit values, 128 bytes a row) and W slice (256 super-block headers of 16
//    bytes + 256 x 32 quant bytes of group c) are copied global -> LDS with buffer_load_dwordx4 ...
//    lds (no registers, no VALU), three stages deep: X two slices ahead, W three.  The main loop
//    issues no other vector-memory operation, so s_waitcnt vmcnt with a static count tracks the
//    copies, and one barrier per slice publishes them.
//  * X rows sit 128 bytes apart with the 16-byte chunk kc of row r at slot kc ^ swz(r),
//    swz(r) = (r ^ (r >> 3 & 3)) & 7: the A-fragment reads (rows r..r+15, one chunk each) hit
//    distinct banks for 32- and 64-bank LDS alike.
//  * B operands: lane (n = lane % 32, g = lane / 32) reads the header and quant bytes 16g..16g+15
//    of group c of its weight row from LDS and dequantises them exactly in fp32 (d*sc*q - dmin*m,
//    one rounding: the reference's dequant value) before rounding to bf16 / fp16; K16 steps 0-3
//    take low nibbles 0-7, 8-15, then high nibbles 0-7, 8-15, and the A operand (X) is read in
//    exactly that element order.  Slice k+1 is dequantised while the MFMAs of slice k run.
//  * The loop reads LDS through inline asm (lds_read16) with explicit lgkmcnt waits: the compiler
//    would otherwise wait for every copy in flight before each LDS read.
// Tiles are numbered in a 1-D grid, M-tile fastest within a column of 256 weight rows, and
// consecutive numbers are placed on one XCD (the dispatcher deals workgroups round-robin over the 8
// XCDs), so the concurrent tiles of an XCD share their columns' weights and their X rows in its L2.
// A launch covers two kinds of columns with their own tile count and first token (TileMap), so the
// host can cut M into one full round of 256-token tiles plus one of shorter tiles where a uniform
// grid would leave the chip part-idle in its last round.  Grids smaller than the chip split K
// across workgroups: each split stores its partial tile, and the split that finishes a tile last
// adds the partials in split order and stores the tile, so results do not vary between runs.
//
// The bf16 variant first rounds X to bf16 (RNE) in a prepass into a stream-ordered temporary; the
// fp16 variant reads X as is.
// qvx_common.hpp (hip_runtime.h) must come first: a standard header included before it stops the
// host stubs of template kernels from being emitted.
#include "qvx_common.hpp"

#include <algorithm>
#include <atomic>
#include <mutex>
#include <utility>

namespace qvx {

namespace gemm {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef int i32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
#define QVX_LDS __attribute__((address_space(3)))

enum { VAR_BF16 = 0, VAR_I8 = 1, VAR_F16 = 2 };

constexpr uint32_t kRsrcWord3 = 0x00020000u;  // raw buffer, 32-bit data (gfx9)
constexpr int kBN = 256;                      // weight rows per workgroup tile
constexpr int kWStage = kBN * 80;             // LDS bytes of one W stage: 256 rows x half a super-block
constexpr int kWQs = kBN * 16;                // ... of which the headers come first, the quant bytes after

// s_waitcnt vmcnt(N), other counters untouched (gfx9 encoding).
template <int N>
__device__ inline void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

template <int OFF = 0>
__device__ inline u32x4 lds_read16(uint32_t addr) {
  u32x4 r;
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "i"(OFF) : "memory");
  return r;
}
// Waits for the LDS reads in flight; the results (the first N of r, then the 4 of w) are operands,
// so no use moves above the wait.
#define QVX_R2(r, i) "+v"(r[i]), "+v"(r[i + 1])
template <int N>
__device__ inline void lds_wait(u32x4* r) {
  static_assert(N == 2 || N == 4 || N == 6 || N == 8, "lds_wait arity");
  if constexpr (N == 2) asm volatile("s_waitcnt lgkmcnt(0)" : QVX_R2(r, 0)::"memory");
  if constexpr (N == 4) asm volatile("s_waitcnt lgkmcnt(0)" : QVX_R2(r, 0), QVX_R2(r, 2)::"memory");
  if constexpr (N == 6) asm volatile("s_waitcnt lgkmcnt(0)" : QVX_R2(r, 0), QVX_R2(r, 2), QVX_R2(r, 4)::"memory");
  if constexpr (N == 8)
    asm volatile("s_waitcnt lgkmcnt(0)" : QVX_R2(r, 0), QVX_R2(r, 2), QVX_R2(r, 4), QVX_R2(r, 6)::"memory");
}
template <int N>
__device__ inline void lds_wait(u32x4* r, u32x4* w) {
  static_assert(N == 4 || N == 8, "lds_wait arity");
  if constexpr (N == 4)
    asm volatile("s_waitcnt lgkmcnt(0)" : QVX_R2(r, 0), QVX_R2(r, 2), QVX_R2(w, 0), QVX_R2(w, 2)::"memory");
  if constexpr (N == 8)
    asm volatile("s_waitcnt lgkmcnt(0)"
                 : QVX_R2(r, 0), QVX_R2(r, 2), QVX_R2(r, 4), QVX_R2(r, 6), QVX_R2(w, 0), QVX_R2(w, 2)::"memory");
}

// Waits as above for the first N of r (N = 0, 2, 4, 6 or 8) and two more results w[0], w[1].
template <int N>
__device__ inline void lds_wait_w2(u32x4* r, u32x4* w) {
  static_assert(N == 0 || N == 2 || N == 4 || N == 6 || N == 8, "lds_wait_w2 arity");
  if constexpr (N == 0) asm volatile("s_waitcnt lgkmcnt(0)" : QVX_R2(w, 0)::"memory");
  if constexpr (N == 2) asm volatile("s_waitcnt lgkmcnt(0)" : QVX_R2(r, 0), QVX_R2(w, 0)::"memory");
  if constexpr (N == 4) asm volatile("s_waitcnt lgkmcnt(0)" : QVX_R2(r, 0), QVX_R2(r, 2), QVX_R2(w, 0)::"memory");
  if constexpr (N == 6)
    asm volatile("s_waitcnt lgkmcnt(0)" : QVX_R2(r, 0), QVX_R2(r, 2), QVX_R2(r, 4), QVX_R2(w, 0)::"memory");
  if constexpr (N == 8)
    asm volatile("s_waitcnt lgkmcnt(0)"
                 : QVX_R2(r, 0), QVX_R2(r, 2), QVX_R2(r, 4), QVX_R2(r, 6), QVX_R2(w, 0)::"memory");
}

__device__ inline void lds_wait8_1(u32x4* r, u32x4* w) {
  asm volatile("s_waitcnt lgkmcnt(0)"
               : "+v"(r[0]), "+v"(r[1]), "+v"(r[2]), "+v"(r[3]), "+v"(r[4]), "+v"(r[5]), "+v"(r[6]), "+v"(r[7]),
                 "+v"(w[0])::"memory");
}

__device__ inline uint32_t xswz(uint32_t r) { return (r ^ ((r >> 3) & 3u)) & 7u; }

// Copy global -> LDS, 16 bytes a lane (a device function of its own: called from a lambda, the target
// builtin makes the host pass drop the kernel's launch stub).
__device__ inline void copy_lds16(__amdgpu_buffer_rsrc_t r, QVX_LDS uint8_t* dst, uint32_t voff, uint32_t soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, dst, 16, voff, soff, 0, 0);
}
// Quant-byte rows of a W stage are 64 bytes apart; 16-byte chunk p of row r sits at slot p ^ qswz(r),
// which keeps the reads of 16 consecutive rows (one chunk each) on distinct banks.
__device__ inline uint32_t qswz(uint32_t r) { return ((r >> 1) ^ (r >> 3)) & 3u; }

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

__device__ inline float ub(uint32_t w, int k) { return (float)((w >> (8 * k)) & 0xFFu); }

// 8 values ds * byte + dm of two dwords of masked codes (one MFMA operand).
template <int VAR>
__device__ inline i32x4_t deq8(uint32_t w0, uint32_t w1, float ds, float dm) {
  i32x4_t o;
  o[0] = (int)pack2<VAR>(__builtin_fmaf(ds, ub(w0, 0), dm), __builtin_fmaf(ds, ub(w0, 1), dm));
  o[1] = (int)pack2<VAR>(__builtin_fmaf(ds, ub(w0, 2), dm), __builtin_fmaf(ds, ub(w0, 3), dm));
  o[2] = (int)pack2<VAR>(__builtin_fmaf(ds, ub(w1, 0), dm), __builtin_fmaf(ds, ub(w1, 1), dm));
  o[3] = (int)pack2<VAR>(__builtin_fmaf(ds, ub(w1, 2), dm), __builtin_fmaf(ds, ub(w1, 3), dm));
  return o;
}

// Shift / mask set that extracts the 6-bit (scale, min) pairs of sub-blocks 2c, 2c+1 from a Q4_K
// header without branches: pair = ((word_a >> sa) & ma) | ((h.w >> sb) & mb), word_a = h.y for the
// scales, h.z for the mins (the min nibbles sit 4 bits higher in h.w).  c is uniform: scalar math.
struct ScaleSel {
  uint32_t sa, ma, sb, mb;
};
__device__ inline ScaleSel scale_sel(int c) {
  const bool hi = c >= 2;
  const uint32_t base = 16u * (uint32_t)(c & 1);
  return ScaleSel{hi ? base + 2u : base, hi ? 0x3030u : 0x3F3Fu, base, hi ? 0x0F0Fu : 0u};
}

// B operands of one weight row for one slice: header h, quant bytes q (16g..16g+15 of group c).
// Low nibbles: ds0 * n - dmin*m0.  High nibbles are kept in place (16 n) and scaled by ds1 / 16,
// an exact power-of-two step, so the fma rounds d*sc*n - dmin*m exactly once.
template <int VAR>
__device__ inline void dequant_row(const u32x4& h, const u32x4& q, const ScaleSel& sel, uint32_t mlo, uint32_t mhi,
                                   i32x4_t (&b)[4]) {
  const uint32_t scp = ((h.y >> sel.sa) & sel.ma) | ((h.w >> sel.sb) & sel.mb);
  const uint32_t mp = ((h.z >> sel.sa) & sel.ma) | ((h.w >> (sel.sb + 4u)) & sel.mb);
  const float d = f16lo(h.x), dmin = f16hi(h.x);
  const float ds0 = d * ub(scp, 0), ds1 = d * ub(scp, 1) * 0.0625f;
  const float dm0 = -(dmin * ub(mp, 0)), dm1 = -(dmin * ub(mp, 1));
  b[0] = deq8<VAR>(q.x & mlo, q.y & mlo, ds0, dm0);
  b[1] = deq8<VAR>(q.z & mlo, q.w & mlo, ds0, dm0);
  b[2] = deq8<VAR>(q.x & mhi, q.y & mhi, ds1, dm1);
  b[3] = deq8<VAR>(q.z & mhi, q.w & mhi, ds1, dm1);
}

// Empty asm that claims to modify v: the value is materialised here, so the compiler cannot sink
// its computation past this point (into the next slice's block).
__device__ inline void pin(i32x4_t& v) { asm volatile("" : "+v"(v)); }

template <int VAR>
__device__ inline f32x16_t mfma32(i32x4_t a, i32x4_t b, f32x16_t c) {
  if constexpr (VAR == VAR_BF16)
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b), c,
                                                   0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a), __builtin_bit_cast(f16x8_t, b), c, 0,
                                                  0, 0);
}

// Shared geometry of one launch.
struct GemmGeo {
  int M, N, K;
  uint32_t row_bytes;  // bytes of one weight row
  int per_split;       // K slices per workgroup along grid z
  uint32_t mask_lo;    // 0x0F0F0F0F and 0xF0F0F0F0, passed at run time: with compile-time masks the
  uint32_t mask_hi;    // compiler re-extracts every nibble (bfe) instead of one AND per dword
  uint32_t m_b0;       // 0x000F000F: bits 0-3 of each 16-bit half (fp16 mantissa bits 0-3)
  uint32_t m_b4;       // 0x00F000F0: bits 4-7 of each 16-bit half (fp16 mantissa bits 4-7)
  float* part = nullptr;     // K-split launches: partial tiles [tile][split][BM * 256]
  uint32_t* cnt = nullptr;   // ... and one arrival counter per tile, zero before the launch
};

// Tile numbering of one launch: columns 0..cols_a-1 hold mt_a tiles from token base_a, columns
// cols_a.. hold mt_b tiles from token base_b (BM tokens a tile, M-tile fastest).
struct TileMap {
  int cols_a, mt_a, base_a, mt_b, base_b;
};

}  // namespace gemm

using namespace gemm;

// Reads A fragments i = 0..MT-1 (32-token tiles 4096 bytes apart) with immediate offsets.
template <int... I>
__device__ inline void read_frags(uint32_t addr, u32x4* a, std::integer_sequence<int, I...>) {
  ((a[I] = lds_read16<4096 * I>(addr)), ...);
}

template <int VAR, int BM>
__global__ __launch_bounds__(512) void k_qgemm_q4k(const uint8_t* __restrict__ W, const uint16_t* __restrict__ X,
                                                   float* __restrict__ Y, GemmGeo geo, TileMap tm) {
  constexpr int MT = BM / 32;         // 32-token A tiles (per wave: all BM tokens)
  constexpr int XI = BM / 64;         // X copies per wave per slice (BM*128 bytes / 8 waves / 1 KB)
  constexpr int WI = 3;               // W copies per wave per half super-block (headers, 2 x quants)
  constexpr int XSTAGE = BM * 128;    // bytes of one X slice
  static_assert(BM % 64 == 0 && BM >= 64 && BM <= 256, "tile size");
  __shared__ __attribute__((aligned(1024))) uint8_t xs[3 * XSTAGE];
  __shared__ __attribute__((aligned(1024))) uint8_t ws[3 * kWStage];

  const int M = geo.M, N = geo.N, K = geo.K;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int ln = lane & 31, g = lane >> 5;
  int n0, m0, tile_id;
  {
    const int nb = (int)gridDim.x;
    int b = (int)blockIdx.x;
    if ((nb & 7) == 0) b = (b & 7) * (nb >> 3) + (b >> 3);  // XCD b % 8 takes a contiguous range
    tile_id = b;
    const int na = tm.cols_a * tm.mt_a;
    if (b < na) {
      n0 = (b / tm.mt_a) * kBN;
      m0 = tm.base_a + (b % tm.mt_a) * BM;
    } else {
      b -= na;
      n0 = (tm.cols_a + b / tm.mt_b) * kBN;
      m0 = tm.base_b + (b % tm.mt_b) * BM;
    }
  }
  const int nsl = K / 64;
  const int kb0 = blockIdx.z * geo.per_split;  // per_split is a multiple of 4: splits start a super-block
  const int kb1 = min(nsl, kb0 + geo.per_split);
  if (kb0 >= kb1 || m0 >= M || n0 >= N) return;

  // Copy descriptors: rows past M or N read as zeros (buffer range check).
  const uint32_t xrow_bytes = (uint32_t)K * 2u;
  const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(X + (size_t)m0 * K), (short)0, (int)((uint32_t)min(BM, M - m0) * xrow_bytes), (int)kRsrcWord3);
  const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(W + (size_t)n0 * geo.row_bytes), (short)0, (int)((uint32_t)min(kBN, N - n0) * geo.row_bytes),
      (int)kRsrcWord3);
  // X copy i of this wave: chunk q = (wave*XI + i)*64 + lane -> row q/8, LDS slot q%8 holds global
  // chunk slot ^ swz(row).
  uint32_t xoff[4];
#pragma unroll
  for (int i = 0; i < XI; ++i) {
    const uint32_t q = (uint32_t)((wave * XI + i) * 64 + lane), r = q >> 3, p = q & 7u;
    xoff[i] = r * xrow_bytes + 16u * (p ^ xswz(r));
  }
  // W copies of this wave's rows 32w..32w+31 for half super-block hb: the 32 headers (lanes 0..31,
  // row 32w + lane, LDS 16 r), then two quant copies (row 32w + 16i + lane/4, LDS slot lane%4 of the
  // row's 64 bytes holds chunk slot ^ qswz(row)).
  const uint32_t woff_h = (uint32_t)(32 * wave + ln) * geo.row_bytes;
  uint32_t woff[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const uint32_t r = (uint32_t)(32 * wave + 16 * i + (lane >> 2)), slot = (uint32_t)lane & 3u;
    woff[i] = r * geo.row_bytes + 16u + 16u * (slot ^ qswz(r));
  }
  QVX_LDS uint8_t* xs_l = (QVX_LDS uint8_t*)xs;
  QVX_LDS uint8_t* ws_l = (QVX_LDS uint8_t*)ws;

  auto issue_x1 = [&](int kb, int i) {
    QVX_LDS uint8_t* dst = xs_l + (kb % 3) * XSTAGE + wave * XI * 1024;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(xr, dst + i * 1024, 16, xoff[i], (uint32_t)kb * 128u, 0, 0);
  };
  auto issue_x = [&](int kb) {
#pragma unroll
    for (int i = 0; i < XI; ++i) issue_x1(kb, i);
  };
  auto issue_w = [&](int hb) {
    QVX_LDS uint8_t* st = ws_l + (hb % 3) * kWStage;
    const uint32_t sbo = (uint32_t)(hb >> 1) * 144u;
    if (lane < 32) __builtin_amdgcn_raw_ptr_buffer_load_lds(wr, st + wave * 512, 16, woff_h, sbo, 0, 0);
#pragma unroll
    for (int i = 0; i < 2; ++i)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(wr, st + kWQs + (2 * wave + i) * 1024, 16, woff[i],
                                               sbo + 64u * (uint32_t)(hb & 1), 0, 0);
  };

  const uint32_t xs_base = (uint32_t)(uintptr_t)xs_l;
  const uint32_t ws_base = (uint32_t)(uintptr_t)ws_l;
  const uint32_t sw = xswz((uint32_t)ln);
  uint32_t a_rel[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    const uint32_t kc = 4u * (uint32_t)(s >> 1) + 2u * (uint32_t)g + (uint32_t)(s & 1);
    a_rel[s] = (uint32_t)ln * 128u + 16u * (kc ^ sw);
  }
  // B: this lane's weight row r = 32w + ln.
  const uint32_t rr = (uint32_t)(32 * wave + ln);
  const uint32_t h_rel = 16u * rr;
  const uint32_t q_rel0 = (uint32_t)kWQs + 64u * rr + 16u * ((uint32_t)g ^ qswz(rr));
  const uint32_t q_rel1 = (uint32_t)kWQs + 64u * rr + 16u * ((2u + (uint32_t)g) ^ qswz(rr));

  f32x16_t acc[8];  // rows >= MT unused
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[i][e] = 0.0f;

  auto read_w = [&](int kb, u32x4 (&r)[2]) {
    const uint32_t st = ws_base + (uint32_t)((kb >> 1) % 3) * kWStage;
    r[0] = lds_read16(st + h_rel);
    r[1] = lds_read16(st + ((kb & 1) ? q_rel1 : q_rel0));
  };

  // Dequantisation of the next slice in 9 pieces of ~9 VALU for this lane's row, placed between the
  // MFMAs by hand: piece 0 = the row's scales, piece 1+u = dwords 2h, 2h+1 of bn[u/2] (h = u%2),
  // converted from quant dword (u/2 % 2)*2 + h, low nibbles for u < 4, high nibbles after.
  // A nibble n is dropped into the mantissa of the fp16 1024 (bits 0x6400) at bit b = 0 or 4 (one
  // bitop3 for the two nibbles of a 16-bit half pair, after a shift for the odd bytes): the half is
  // exactly 1024 + 2^b n, and v_fma_mix_f32 evaluates (ds / 2^b) * (1024 + 2^b n) +
  // (dm - 1024 ds / 2^b) = ds * n + dm with one rounding (the bias itself rounds once, ~2^-14 ds:
  // far below the bf16 / fp16 rounding that follows).  Byte k of a quant dword:
  //   low nibble,  k even: (w      & 0x000F000F) -> n       low nibble,  k odd: (w >> 4 & 0x00F000F0) -> 16 n
  //   high nibble, k even: (w      & 0x00F000F0) -> 16 n    high nibble, k odd: (w >> 8 & 0x00F000F0) -> 16 n
  struct DeqState {
    u32x4 h, q;
    float s[3], b[3];  // scale, bias: low even, low odd, high
    ScaleSel sel;
  };
  const uint32_t k1024 = 0x64006400u;  // two fp16 1024.0
  auto piece = [&](int p, DeqState& st, i32x4_t (&bn)[4]) {
    if (p == 0) {
      const u32x4& h = st.h;
      const uint32_t scp = ((h.y >> st.sel.sa) & st.sel.ma) | ((h.w >> st.sel.sb) & st.sel.mb);
      const uint32_t mp = ((h.z >> st.sel.sa) & st.sel.ma) | ((h.w >> (st.sel.sb + 4u)) & st.sel.mb);
      const float d = f16lo(h.x), dmin = f16hi(h.x);
      const float ds0 = d * ub(scp, 0), ds1 = d * ub(scp, 1);
      const float dm0 = -(dmin * ub(mp, 0)), dm1 = -(dmin * ub(mp, 1));
      st.s[0] = ds0;
      st.s[1] = ds0 * 0.0625f;
      st.s[2] = ds1 * 0.0625f;
      st.b[0] = __builtin_fmaf(-1024.0f, ds0, dm0);
      st.b[1] = __builtin_fmaf(-64.0f, ds0, dm0);
      st.b[2] = __builtin_fmaf(-64.0f, ds1, dm1);
    } else {
      const int u = p - 1, sp = u >> 1, hh = u & 1, w = (sp & 1) * 2 + hh;
      const uint32_t src = w == 0 ? st.q.x : w == 1 ? st.q.y : w == 2 ? st.q.z : st.q.w;
      const bool lo = sp < 2;
      const int ke = lo ? 0 : 2, ko = lo ? 1 : 2;
      const uint32_t e = __builtin_amdgcn_bitop3_b32(src, lo ? geo.m_b0 : geo.m_b4, k1024, 0xEA);
      const uint32_t o = __builtin_amdgcn_bitop3_b32(src >> (lo ? 4 : 8), geo.m_b4, k1024, 0xEA);
      const half2_t he = __builtin_bit_cast(half2_t, e), ho = __builtin_bit_cast(half2_t, o);
      bn[sp][2 * hh] = (int)pack2<VAR>(__builtin_fmaf((float)he.x, st.s[ke], st.b[ke]),
                                       __builtin_fmaf((float)ho.x, st.s[ko], st.b[ko]));
      bn[sp][2 * hh + 1] = (int)pack2<VAR>(__builtin_fmaf((float)he.y, st.s[ke], st.b[ke]),
                                           __builtin_fmaf((float)ho.y, st.s[ko], st.b[ko]));
      pin(bn[sp]);
    }
  };

  // A fragments go through a ring of two groups of four 32-token tiles (NG groups per slice, group G
  // = step G / (MT/4), tiles 4 (G % (MT/4)) ..+3); a group's reads are issued one group ahead, so four
  // MFMAs (eight with the SIMD's other wave) cover their latency.
  constexpr int GPS = MT / 4 > 0 ? MT / 4 : 1;  // groups per K16 step
  constexpr int GT = MT / GPS;                  // tiles per group
  constexpr int NG = 4 * GPS;                   // groups per slice
  auto read_group = [&](uint32_t xb, int G, u32x4 (&r)[8]) {
    const uint32_t base = xb + a_rel[G / GPS] + 4096u * (uint32_t)(GT * (G % GPS));
    read_frags(base, r, std::make_integer_sequence<int, GT>{});
  };
  // Dequantisation pieces of slice kb+1 go after the MFMAs of groups 1..NG-1: piece p after slot
  // p * NS / 9 of those NS = GT (NG - 1) slots.
  constexpr int NS = GT * (NG - 1);

  // One slice: group 0's fragments were read during the previous slice.  Group 0 also issues the
  // X(kb+2) copies (one after each MFMA) and the LDS reads of this lane's W(kb+1) header and quant
  // bytes; the barrier that publishes X(kb+1) and frees stage kb%3 comes once every fragment of
  // slice kb is in registers (before the last group), and W(kb/2+2) is issued right after it on even
  // slices.
  auto slice = [&](int kb, const i32x4_t (&bc)[4], i32x4_t (&bn)[4], u32x4 (&a)[2][8]) {
    const uint32_t xb = xs_base + (uint32_t)(kb % 3) * XSTAGE;
    DeqState st;
    st.sel = scale_sel((kb + 1) & 3);
    const int kx = min(kb + 2, kb1 - 1);
#pragma unroll
    for (int G = 0; G < NG; ++G) {
      u32x4(&cur)[8] = a[G & 1];
      u32x4(&nxt)[8] = a[(G + 1) & 1];
      if (G == 1) {
        u32x4 w2[2] = {st.h, st.q};
        lds_wait_w2<GT>(cur, w2);
        st.h = w2[0];
        st.q = w2[1];
      } else {
        lds_wait<GT>(cur);
      }
      if (G == NG - 1) {
        if (kb + 1 < kb1) {
          // X(kb+1) was copied during group 0 of slice kb-1; younger copies, which may still fly:
          // W of the sync of slice kb-1 (odd kb) and X(kb+2) (group 0 of this slice).
          if ((kb & 1) && kb + 3 < kb1)
            wait_vm<WI + XI>();
          else
            wait_vm<XI>();
          __builtin_amdgcn_s_barrier();
          if (!(kb & 1) && kb + 4 < kb1) issue_w((kb >> 1) + 2);
          read_group(xs_base + (uint32_t)((kb + 1) % 3) * XSTAGE, 0, nxt);
        }
      } else {
        read_group(xb, G + 1, nxt);
      }
      if (G == 0) {
        u32x4 w2[2];
        read_w(kb + 1, w2);
        st.h = w2[0];
        st.q = w2[1];
      }
      __builtin_amdgcn_sched_barrier(0);
      const int s = G / GPS;
#pragma unroll
      for (int t = 0; t < GT; ++t) {
        acc[GT * (G % GPS) + t] = mfma32<VAR>(__builtin_bit_cast(i32x4_t, cur[t]), bc[s], acc[GT * (G % GPS) + t]);
        if (G == 0 && t < XI) issue_x1(kx, t);
        if (G > 0) {
          const int slot = GT * (G - 1) + t;
#pragma unroll
          for (int p = 0; p < 9; ++p)
            if (p * NS / 9 == slot) piece(p, st, bn);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  };

  issue_w(kb0 >> 1);
  issue_x(kb0);
  wait_vm<0>();
  __builtin_amdgcn_s_barrier();
  if (kb0 + 2 < kb1) issue_w((kb0 >> 1) + 1);
  issue_x(min(kb0 + 1, kb1 - 1));

  u32x4 a[2][8];
  read_group(xs_base + (uint32_t)(kb0 % 3) * XSTAGE, 0, a[0]);
  i32x4_t b0[4], b1[4];
  {
    u32x4 wq[2];
    read_w(kb0, wq);
    lds_wait_w2<0>(nullptr, wq);
    dequant_row<VAR>(wq[0], wq[1], scale_sel(kb0 & 3), geo.mask_lo, geo.mask_hi, b0);
  }

  int kb = kb0;
  for (; kb + 1 < kb1; kb += 2) {
    slice(kb, b0, b1, a);
    slice(kb + 1, b1, b0, a);
  }
  if (kb < kb1) slice(kb, b0, b1, a);
  wait_vm<0>();

  // K split: the split that finishes a tile last sums the partials in split order and stores it.
  if (gridDim.z > 1) {
    float v[MT * 16];
#pragma unroll
    for (int a = 0; a < MT * 16; ++a) v[a] = acc[a >> 4][a & 15];
    if (!split_k_last<MT * 16, 512>(v, geo.part + (size_t)tile_id * gridDim.z * (MT * 16 * 512), geo.cnt + tile_id,
                                    (int)gridDim.z, (int)blockIdx.z, tid, reinterpret_cast<int*>(xs)))
      return;
#pragma unroll
    for (int a = 0; a < MT * 16; ++a) acc[a >> 4][a & 15] = v[a];
  }

#pragma unroll
  for (int i = 0; i < MT; ++i) {
    const int n = n0 + 32 * wave + ln;
    if (n >= N) continue;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int m = m0 + 32 * i + 8 * (e >> 2) + 4 * g + (e & 3);
      if (m < M) Y[(size_t)m * N + n] = acc[i][e];
    }
  }
}

// ---- 4-wave form: one wave per SIMD, BM tokens x 64 weight rows a wave ------------------------------
// k_qgemm_q4kq<VAR, BM>: a BM-token x 256-row tile per 256-thread workgroup; wave w owns weight rows
// 64w..64w+63 and all BM tokens (BM/32 x 2 tiles of v_mfma_f32_32x32x16_*, the accumulators in the
// accumulation registers).  The product runs BM = 256 (at BM = 128, with or without a K split, this
// form measured 8-16 % slower than the 8-wave kernel on the same tiles, which keeps them).  Each weight element is dequantised once per
// workgroup, by the wave that owns its row, and each wave reads every X fragment of a slice: per K16
// step BM/32 A fragments and two B fragments for BM/16 MFMAs, half the LDS traffic per MFMA of the
// 8-wave kernel above, whose waves each read all BM tokens' fragments for 32 rows.  K advances in
// 64-element slices (group c of a super-block) through three stages filled by buffer_load ... lds
// two slices ahead: X rows (128 bytes, chunks swizzled as above), the 256 super-block headers (16
// bytes each) and the 256 rows' 32 quant bytes of group c (the two 16-byte halves of row r swapped
// when bit 3 of r is set, so the reads of 16 consecutive rows hit distinct banks).  Lane (n, g) of
// row tile t takes the header and quant bytes 16g..16g+15 of row 64w + 32t + n once per slice and
// makes the B operands of the four K16 steps from them (low nibbles 0-7, 8-15, high nibbles 0-7,
// 8-15 -- the element order of the 8-wave kernel, and the A fragments are read in that order), one
// step ahead, between the MFMAs, with the 8-wave kernel's main-loop arithmetic (the fp16-1024
// mantissa insertion and v_fma_mix evaluation).  One barrier per slice, before its last step: every
// wave has then read the slice's X, so its stage is refilled during that step, and has waited for
// its copies of the next slice, whose headers and quant bytes it reads right after the barrier.
template <int VAR, int BM>
__global__ __launch_bounds__(256) void k_qgemm_q4kq(const uint8_t* __restrict__ W, const uint16_t* __restrict__ X,
                                                    float* __restrict__ Y, GemmGeo geo, TileMap tm) {
  static_assert(BM == 256 || BM == 128, "tile tokens");
  constexpr int NST = 3;
  constexpr int TT = BM / 32;           // 32-token tiles of a wave
  constexpr int NK = 2 * TT;            // MFMAs a K16 step
  constexpr int XST = BM * 128;         // X rows of a slice
  constexpr int HST = kBN * 16;         // the tile's super-block headers
  constexpr int QST = kBN * 32;         // quant bytes of group c of the tile's rows
  constexpr int STB = XST + HST + QST;  // one stage
  constexpr int XC = BM / 32;           // X copies per wave per slice
  constexpr int CPW = XC + 3;           // copies per wave per slice: X, 1 header, 2 quant
  // slots within a step: the B operand pieces of the next step; in the last step the wait for the
  // next slice's headers and quant bytes, its first A fragments, its scales
  constexpr int RW = NK >= 16 ? 3 : 2;
  auto piece_slot = [](int p) { return NK >= 16 ? 8 + 2 * p : NK - 4 + p; };
  __shared__ __attribute__((aligned(1024))) uint8_t lds[NST * STB];
  const int M = geo.M, N = geo.N, K = geo.K;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int ln = lane & 31, g = lane >> 5;
  int n0, m0;
  {
    const int nb = (int)gridDim.x;
    int b = (int)blockIdx.x;
    if ((nb & 7) == 0) b = (b & 7) * (nb >> 3) + (b >> 3);  // XCD b % 8 takes a contiguous range
    const int na = tm.cols_a * tm.mt_a;
    if (b < na) {
      n0 = (b / tm.mt_a) * kBN;
      m0 = tm.base_a + (b % tm.mt_a) * BM;
    } else {
      b -= na;
      n0 = (tm.cols_a + b / tm.mt_b) * kBN;
      m0 = tm.base_b + (b % tm.mt_b) * BM;
    }
  }
  const int kb0 = 0, NJ = K / 64;  // no K split: the plan runs this kernel on grids that fill the chip
  if (m0 >= M || n0 >= N) return;
  const uint32_t xrow_bytes = (uint32_t)K * 2u;
  const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(X + (size_t)m0 * K), (short)0, (int)((uint32_t)min(BM, M - m0) * xrow_bytes), (int)kRsrcWord3);
  const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(W + (size_t)n0 * geo.row_bytes), (short)0, (int)((uint32_t)min(kBN, N - n0) * geo.row_bytes),
      (int)kRsrcWord3);
  // Copy offsets of this wave.  X copy i: chunk q = (XC w + i) * 64 + lane -> row q / 8, LDS slot
  // q % 8 holds global chunk slot ^ xswz(row).  Header copy: row 64w + lane.  Quant copy i: LDS slot
  // q = (2w + i) * 64 + lane -> row q / 2, half q % 2 holds global half (q % 2) ^ (row >> 3 & 1).
  uint32_t xoff[XC], qoff[2];
#pragma unroll
  for (int i = 0; i < XC; ++i) {
    const uint32_t q = (uint32_t)((XC * wave + i) * 64 + lane), r = q >> 3, p = q & 7u;
    xoff[i] = r * xrow_bytes + 16u * (p ^ xswz(r));
  }
  const uint32_t hoff = (uint32_t)(64 * wave + lane) * geo.row_bytes;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const uint32_t q = (uint32_t)((2 * wave + i) * 64 + lane), r = q >> 1;
    qoff[i] = r * geo.row_bytes + 16u + 16u * ((q & 1u) ^ ((r >> 3) & 1u));
  }
  QVX_LDS uint8_t* lds_l = (QVX_LDS uint8_t*)lds;
  const uint32_t lds_base = (uint32_t)(uintptr_t)lds_l;
  auto copy1 = [&](int j, int i) {  // copy i (0..CPW-1) of slice kb0 + j
    QVX_LDS uint8_t* st = lds_l + (j % NST) * STB;
    const int kb = kb0 + j;
    const uint32_t sbo = (uint32_t)(kb >> 2) * 144u;
    if (i < XC)
      copy_lds16(xr, st + (XC * wave + i) * 1024, xoff[i], (uint32_t)kb * 128u);
    else if (i == XC)
      copy_lds16(wr, st + XST + wave * 1024, hoff, sbo);
    else
      copy_lds16(wr, st + XST + HST + (2 * wave + i - XC - 1) * 1024, qoff[i - XC - 1], sbo + 32u * (uint32_t)(kb & 3));
  };
  // A fragment reads: step s takes chunk kc = 2g + (s & 1) + 4 (s >> 1) of token row 32 tt + ln.
  const uint32_t sw = xswz((uint32_t)ln);
  uint32_t a_rel[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    const uint32_t kc = 2u * (uint32_t)g + (uint32_t)(s & 1) + 4u * (uint32_t)(s >> 1);
    a_rel[s] = (uint32_t)ln * 128u + 16u * (kc ^ sw);
  }
  auto read_a = [&](int j, int s, int tt) -> u32x4 {
    const uint32_t a = lds_base + (uint32_t)(j % NST) * STB + a_rel[s];
    switch (tt) {
      case 0: return lds_read16<0>(a);
      case 1: return lds_read16<4096>(a);
      case 2: return lds_read16<8192>(a);
      case 3: return lds_read16<12288>(a);
      case 4: return lds_read16<16384>(a);
      case 5: return lds_read16<20480>(a);
      case 6: return lds_read16<24576>(a);
      default: return lds_read16<28672>(a);
    }
  };
  // B: rows 64w + 32t + ln (t = 0, 1): header and quant half g (swapped as copied).
  const uint32_t h_rel = (uint32_t)XST + 16u * (uint32_t)(64 * wave + ln);
  const uint32_t q_rel = (uint32_t)(XST + HST) + 32u * (uint32_t)(64 * wave + ln) +
                         16u * ((uint32_t)g ^ (((uint32_t)ln >> 3) & 1u));
  struct Raw {
    u32x4 h[2], q[2];
  };
  auto read_raw = [&](int j, Raw& r) {
    const uint32_t st = lds_base + (uint32_t)(j % NST) * STB;
    r.h[0] = lds_read16<0>(st + h_rel);
    r.h[1] = lds_read16<512>(st + h_rel);
    r.q[0] = lds_read16<0>(st + q_rel);
    r.q[1] = lds_read16<1024>(st + q_rel);
  };
  // Scale / bias of one row for the slice's group: low nibbles even bytes, odd bytes, high nibbles.
  struct Sc {
    float s[3], b[3];
  };
  auto scales = [&](const u32x4& h, const ScaleSel& sel, Sc& o) {
    const uint32_t scp = ((h.y >> sel.sa) & sel.ma) | ((h.w >> sel.sb) & sel.mb);
    const uint32_t mp = ((h.z >> sel.sa) & sel.ma) | ((h.w >> (sel.sb + 4u)) & sel.mb);
    const float d = f16lo(h.x), dmin = f16hi(h.x);
    const float ds0 = d * ub(scp, 0), ds1 = d * ub(scp, 1);
    const float dm0 = -(dmin * ub(mp, 0)), dm1 = -(dmin * ub(mp, 1));
    o.s[0] = ds0;
    o.s[1] = ds0 * 0.0625f;
    o.s[2] = ds1 * 0.0625f;
    o.b[0] = __builtin_fmaf(-1024.0f, ds0, dm0);
    o.b[1] = __builtin_fmaf(-64.0f, ds0, dm0);
    o.b[2] = __builtin_fmaf(-64.0f, ds1, dm1);
  };
  const uint32_t k1024 = 0x64006400u;  // two fp16 1024.0
  // Half (dwords 2 hh, 2 hh + 1) of the B operand of step s from quant dword src (see the 8-wave kernel).
  auto deq_half = [&](uint32_t src, int s, const Sc& c, i32x4_t& bo, int hh) {
    const bool lo = s < 2;
    const int ke = lo ? 0 : 2, ko = lo ? 1 : 2;
    const uint32_t e = __builtin_amdgcn_bitop3_b32(src, lo ? geo.m_b0 : geo.m_b4, k1024, 0xEA);
    const uint32_t o = __builtin_amdgcn_bitop3_b32(src >> (lo ? 4 : 8), geo.m_b4, k1024, 0xEA);
    const half2_t he = __builtin_bit_cast(half2_t, e), ho = __builtin_bit_cast(half2_t, o);
    bo[2 * hh] = (int)pack2<VAR>(__builtin_fmaf((float)he.x, c.s[ke], c.b[ke]), __builtin_fmaf((float)ho.x, c.s[ko], c.b[ko]));
    bo[2 * hh + 1] =
        (int)pack2<VAR>(__builtin_fmaf((float)he.y, c.s[ke], c.b[ke]), __builtin_fmaf((float)ho.y, c.s[ko], c.b[ko]));
  };
  // piece p (0..3) of step s's B operands: row tile p / 2, half p % 2 (quant dword (s & 1) * 2 + p % 2)
  auto deq_piece = [&](const Raw& r, const Sc (&c)[2], int s, int p, i32x4_t (&bo)[2]) {
    const int t = p >> 1, hh = p & 1, w = (s & 1) * 2 + hh;
    const u32x4& q = r.q[t];
    const uint32_t src = w == 0 ? q.x : w == 1 ? q.y : w == 2 ? q.z : q.w;
    deq_half(src, s, c[t], bo[t], hh);
    pin(bo[t]);
  };

  f32x16_t acc[TT][2];
#pragma unroll
  for (int i = 0; i < TT; ++i)
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][t][e] = 0.0f;

  // prologue: slices 0..2 in flight, slice 0's operands of step 0 in registers
#pragma unroll
  for (int j = 0; j < NST; ++j)
    if (j < NJ)
#pragma unroll
      for (int i = 0; i < CPW; ++i) copy1(j, i);
  if (NJ > 2)
    wait_vm<2 * CPW>();
  else if (NJ > 1)
    wait_vm<CPW>();
  else
    wait_vm<0>();
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_sched_barrier(0);
  u32x4 a[2][8];  // entries >= TT unused
  i32x4_t bf[2][2];
  Raw raw;
  Sc sc[2];
  read_raw(0, raw);
#pragma unroll
  for (int tt = 0; tt < TT; ++tt) a[0][tt] = read_a(0, 0, tt);
  asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(raw.h[0]), "+v"(raw.h[1]), "+v"(raw.q[0]), "+v"(raw.q[1]) ::"memory");
  lds_wait<TT>(a[0]);
  {
    const ScaleSel sel = scale_sel(kb0 & 3);
    scales(raw.h[0], sel, sc[0]);
    scales(raw.h[1], sel, sc[1]);
#pragma unroll
    for (int p = 0; p < 4; ++p) deq_piece(raw, sc, 0, p, bf[0]);
  }
  __builtin_amdgcn_sched_barrier(0);

  // One slice.  REFILL: the copies of slice j + 3 are issued after the barrier; MORE: slice j + 1
  // follows (its operands are read and its step-0 B operands made during the last step); YOUNG: the
  // copies of slice j + 2 were issued (the barrier's wait leaves them in flight).
  auto slice = [&]<bool REFILL, bool MORE, bool YOUNG>(int j) {
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      u32x4(&cur)[8] = a[s & 1];
      u32x4(&nxt)[8] = a[(s + 1) & 1];
      i32x4_t(&bc)[2] = bf[s & 1];
      i32x4_t(&bn)[2] = bf[(s + 1) & 1];
      if (s == 3) {
        if constexpr (YOUNG)
          wait_vm<CPW>();
        else
          wait_vm<0>();
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (MORE) read_raw(j + 1, raw);
      }
#pragma unroll
      for (int k = 0; k < NK; ++k) {
        const int tt = k >> 1, t = k & 1;
        acc[tt][t] = mfma32<VAR>(__builtin_bit_cast(i32x4_t, cur[tt]), bc[t], acc[tt][t]);
        if (s < 3) {
          if (k < TT) nxt[k] = read_a(j, s + 1, k);
#pragma unroll
          for (int p = 0; p < 4; ++p)
            if (k == piece_slot(p)) deq_piece(raw, sc, s + 1, p, bn);
        } else {
          if constexpr (REFILL)
            if (k < CPW) copy1(j + NST, k);
          if constexpr (MORE) {
            if (k == RW)
              asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(raw.h[0]), "+v"(raw.h[1]), "+v"(raw.q[0]), "+v"(raw.q[1])::"memory");
            if (k > RW && k <= RW + TT) nxt[k - RW - 1] = read_a(j + 1, 0, k - RW - 1);
            if (k == RW + 2) {
              const ScaleSel sel = scale_sel((kb0 + j + 1) & 3);
              scales(raw.h[0], sel, sc[0]);
              scales(raw.h[1], sel, sc[1]);
            }
#pragma unroll
            for (int p = 0; p < 4; ++p)
              if (k == piece_slot(p)) deq_piece(raw, sc, 0, p, bn);
          }
        }
        __builtin_amdgcn_sched_barrier(0);
      }
      if (s < 3 || MORE) lds_wait<TT>(nxt);
    }
  };
  int j = 0;
  for (; j + NST < NJ; ++j) slice.template operator()<true, true, true>(j);
  for (; j + 2 < NJ; ++j) slice.template operator()<false, true, true>(j);
  for (; j + 1 < NJ; ++j) slice.template operator()<false, true, false>(j);
  slice.template operator()<false, false, false>(j);

#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int n = n0 + 64 * wave + 32 * t + ln;
    if (n >= N) continue;
#pragma unroll
    for (int i = 0; i < TT; ++i)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int m = m0 + 32 * i + 8 * (e >> 2) + 4 * g + (e & 3);
        if (m < M) Y[(size_t)m * N + n] = acc[i][t][e];
      }
  }
}

// ---- Q6_K on the same pipeline --------------------------------------------------------------------
// k_qgemm_q6k8<VAR>: the structure of k_qgemm_q4k<VAR, 128> (8 waves, wave w = weight rows
// 32w..32w+31 of a 256-row tile and all 128 tokens; X slices three stages deep; B operands
// dequantised in registers while the MFMAs run) for Q6_K weights.  Per super-block the tile's raw
// blocks are staged whole, two stages: each row's dword-aligned window (the block's 210 bytes after
// up to 2 lead bytes: 14 chunks of 16 bytes), copied by 7 LDS-DMA copies per wave, copy k moving
// chunks 2k, 2k+1 of the wave's 32 rows (lane l: row l / 2, chunk 2k + l % 2), so the wave's part of
// a stage is [k][row][2 chunks] (each wave copies and reads only its own rows).  Slice kb covers
// elements 64 (kb % 4) .. +63 of a block; for its half n = (kb / 2) % 2 lane (row, g) reads ql
// bytes 64n + 16g .. +15 (QA) and 64n + 32 + 16g .. +15 (QB), qh bytes 32n + 16g .. +15 (H), the
// half's 8 scale bytes and d, once per half, and builds both slices of the half from them
// (i = 0..15, P = kb % 2):
//   element 16g + i      = (P ? QA_i >> 4 : QA_i & 15) | (H_i bits 4P, 4P+1) << 4,   scale sc[8n + g + 4P]
//   element 32 + 16g + i = (P ? QB_i >> 4 : QB_i & 15) | (H_i bits 4P+2, 4P+3) << 4, scale sc[8n + g + 2 + 4P]
// -- the element order of the Q4_K kernel's B operands and X fragments.  A 6-bit code c goes into the
// mantissa of the fp16 1024 (exactly 1024 + c) and v_fma_mix_f32 gives ds (1024 + c) - 1056 ds =
// ds (c - 32) (ds = d * sc, exact in fp32; the bias rounds once, ~2^-14 ds) before the bf16 / fp16
// rounding of the operand.
struct Q6kGeo {
  int M, N, K;
  uint32_t row_bytes;  // a multiple of 4 (an even number of blocks): every row's blocks share one alignment
  int per_split;       // K slices per split, a multiple of 4
  uint32_t m0f, m30, mff;  // 0x0F0F0F0F, 0x30303030, 0x00FF00FF, at run time (see GemmGeo)
  float* part;
  uint32_t* cnt;
};
constexpr int kQ6Win = 224;              // LDS bytes of a row's block window (14 chunks)
constexpr int kQ6WStage = kBN * kQ6Win;  // one super-block of a 256-row tile: 57344 bytes
constexpr int kQ6Copies = kQ6Win / 32;   // 16-byte copies per wave per super-block: 7

typedef uint32_t q6u32x2 __attribute__((ext_vector_type(2)));
// LDS reads (the compiler does not track them; see lds_read16): 8 and 4 bytes.
template <int OFF>
__device__ inline q6u32x2 lds_read8(uint32_t addr) {
  q6u32x2 r;
  asm volatile("ds_read_b64 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "i"(OFF) : "memory");
  return r;
}
template <int OFF>
__device__ inline uint32_t lds_read4(uint32_t addr) {
  uint32_t r;
  asm volatile("ds_read_b32 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "i"(OFF) : "memory");
  return r;
}
// A half's raw window reads as issued (untouched until q6k_wait: a copy would read them early).
struct Q6kRaw {
  u32x4 qa, qb, h;
  uint32_t qa4, qb4, h4, sc2, d;
  q6u32x2 sc;
};
// Issues the reads of half n of the lane's row window.  row: LDS byte address of the row's chunk 0
// (the wave's part of the stage + 32 * row); chunk c sits at row + 1024 (c / 2) + 16 (c % 2), and the
// chunk after an even chunk 16 bytes on, after an odd one 1008 bytes on (nx = 16 or 1008 for lane K
// half g = 0 or 1).  QA is chunk 4n + g and the next chunk's first dword, QB chunk 4n + 2 + g (+1024),
// H (qh bytes 32n + 16g: block dwords 32 + 8n + 4g) chunk 8 + 2n + g, the scales block dwords
// 48 + 2n .. +2 and d dword 52 (chunks 12 and 13).
__device__ inline void q6k_issue(uint32_t row, int n, int g, Q6kRaw& w) {
  const uint32_t nx = g ? 1008u : 16u;
  const uint32_t a1 = row + 2048u * (uint32_t)n + 16u * (uint32_t)g, a1n = a1 + nx;
  const uint32_t a2 = row + 1024u * (uint32_t)(4 + n) + 16u * (uint32_t)g, a2n = a2 + nx;
  const uint32_t a3 = row + 6144u + 8u * (uint32_t)n;
  w.qa = lds_read16<0>(a1);
  w.qa4 = lds_read4<0>(a1n);
  w.qb = lds_read16<1024>(a1);
  w.qb4 = lds_read4<1024>(a1n);
  w.h = lds_read16<0>(a2);
  w.h4 = lds_read4<0>(a2n);
  w.sc = lds_read8<0>(a3);
  w.sc2 = lds_read4<8>(a3);
  w.d = lds_read4<6160>(row);
}
// Waits for the reads of q6k_issue and the 4 A fragments r (all are operands: no use moves above it).
__device__ inline void q6k_wait(u32x4* r, Q6kRaw& w) {
  asm volatile("s_waitcnt lgkmcnt(0)"
               : "+v"(r[0]), "+v"(r[1]), "+v"(r[2]), "+v"(r[3]), "+v"(w.qa), "+v"(w.qb), "+v"(w.h), "+v"(w.qa4),
                 "+v"(w.qb4), "+v"(w.h4), "+v"(w.sc), "+v"(w.sc2), "+v"(w.d)::"memory");
}
__device__ inline void q6k_wait(Q6kRaw& w) {
  asm volatile("s_waitcnt lgkmcnt(0)"
               : "+v"(w.qa), "+v"(w.qb), "+v"(w.h), "+v"(w.qa4), "+v"(w.qb4), "+v"(w.h4), "+v"(w.sc), "+v"(w.sc2),
                 "+v"(w.d)::"memory");
}
// The half realigned by the block's lead bytes sh (0 or 2): 16 QA, QB and H bytes, 8 scale bytes, d.
struct Q6kHalf {
  uint32_t qa[4], qb[4], h[4], s[2];
  float d;
};
__device__ inline void q6k_align(const Q6kRaw& w, uint32_t sh, Q6kHalf& o) {
  o.qa[0] = align_bytes(w.qa.y, w.qa.x, sh);
  o.qa[1] = align_bytes(w.qa.z, w.qa.y, sh);
  o.qa[2] = align_bytes(w.qa.w, w.qa.z, sh);
  o.qa[3] = align_bytes(w.qa4, w.qa.w, sh);
  o.qb[0] = align_bytes(w.qb.y, w.qb.x, sh);
  o.qb[1] = align_bytes(w.qb.z, w.qb.y, sh);
  o.qb[2] = align_bytes(w.qb.w, w.qb.z, sh);
  o.qb[3] = align_bytes(w.qb4, w.qb.w, sh);
  o.h[0] = align_bytes(w.h.y, w.h.x, sh);
  o.h[1] = align_bytes(w.h.z, w.h.y, sh);
  o.h[2] = align_bytes(w.h.w, w.h.z, sh);
  o.h[3] = align_bytes(w.h4, w.h.w, sh);
  o.s[0] = align_bytes(w.sc.y, w.sc.x, sh);
  o.s[1] = align_bytes(w.sc2, w.sc.y, sh);
  o.d = f16lo(align_bytes(0u, w.d, sh));
}
// Stages the window at byte offset soff (dword aligned, the same for every row) of this wave's 32
// rows: copy k, lane l moves chunk 2k + l % 2 of row l / 2 (voff = that row's offset + 16 (l % 2),
// 16 bytes from a dword-aligned address) to byte 1024k + 16l of the wave's part of the stage.  Rows
// past the tile's buffer range read as zeros.
__device__ __attribute__((always_inline)) inline void q6k_copy(__amdgpu_buffer_rsrc_t wr, QVX_LDS uint8_t* dst,
                                                              uint32_t voff, uint32_t soff, int k) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(wr, dst + 1024 * k, 16, voff, soff + 32u * (uint32_t)k, 0, 0);
}
__device__ __attribute__((always_inline)) inline void q6k_stage(__amdgpu_buffer_rsrc_t wr, QVX_LDS uint8_t* dst,
                                                               uint32_t voff, uint32_t soff) {
#pragma unroll
  for (int k = 0; k < kQ6Copies; ++k) q6k_copy(wr, dst, voff, soff, k);
}

template <int VAR>
__global__ __launch_bounds__(512) void k_qgemm_q6k8(const uint8_t* __restrict__ W, const uint16_t* __restrict__ X,
                                                    float* __restrict__ Y, Q6kGeo geo, TileMap tm) {
  constexpr int BM = 128;
  constexpr int MT = BM / 32, XI = BM / 64, XSTAGE = BM * 128;
  constexpr int GT = MT, NG = 4, NS = GT * (NG - 1), NP = 10;  // one 4-tile A group per K16 step
  __shared__ __attribute__((aligned(1024))) uint8_t xs[3 * XSTAGE];
  __shared__ __attribute__((aligned(1024))) uint8_t ws[2 * kQ6WStage];

  const int M = geo.M, N = geo.N, K = geo.K;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int ln = lane & 31, g = lane >> 5;
  int n0, m0, tile_id;
  {
    const int nb = (int)gridDim.x;
    int b = (int)blockIdx.x;
    if ((nb & 7) == 0) b = (b & 7) * (nb >> 3) + (b >> 3);  // XCD b % 8 takes a contiguous range
    tile_id = b;
    const int na = tm.cols_a * tm.mt_a;
    if (b < na) {
      n0 = (b / tm.mt_a) * kBN;
      m0 = tm.base_a + (b % tm.mt_a) * BM;
    } else {
      b -= na;
      n0 = (tm.cols_a + b / tm.mt_b) * kBN;
      m0 = tm.base_b + (b % tm.mt_b) * BM;
    }
  }
  const int nsl = K / 64;
  const int kb0 = blockIdx.z * geo.per_split;  // a multiple of 4: splits start a super-block
  const int kb1 = min(nsl, kb0 + geo.per_split);
  const int sb_end = kb1 >> 2;

  const uint32_t xrow_bytes = (uint32_t)K * 2u;
  const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(X + (size_t)m0 * K), (short)0, (int)((uint32_t)min(BM, M - m0) * xrow_bytes), (int)kRsrcWord3);
  const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(W + (size_t)n0 * geo.row_bytes), (short)0, (int)((uint32_t)min(kBN, N - n0) * geo.row_bytes),
      (int)kRsrcWord3);
  uint32_t xoff[XI];
#pragma unroll
  for (int i = 0; i < XI; ++i) {
    const uint32_t q = (uint32_t)((wave * XI + i) * 64 + lane), r = q >> 3, p = q & 7u;
    xoff[i] = r * xrow_bytes + 16u * (p ^ xswz(r));
  }
  const uint32_t voff = (uint32_t)(32 * wave + (lane >> 1)) * geo.row_bytes + 16u * (uint32_t)(lane & 1);
  QVX_LDS uint8_t* xs_l = (QVX_LDS uint8_t*)xs;
  QVX_LDS uint8_t* ws_l = (QVX_LDS uint8_t*)ws;
  auto issue_x1 = [&](int kb, int i) {
    QVX_LDS uint8_t* dst = xs_l + (kb % 3) * XSTAGE + wave * XI * 1024;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(xr, dst + i * 1024, 16, xoff[i], (uint32_t)kb * 128u, 0, 0);
  };
  auto issue_x = [&](int kb) {
#pragma unroll
    for (int i = 0; i < XI; ++i) issue_x1(kb, i);
  };
  auto issue_w = [&](int sb) {
    q6k_stage(wr, ws_l + (sb & 1) * kQ6WStage + wave * 32 * kQ6Win, voff, (uint32_t)(sb * 210) & ~3u);
  };
  // After the prologue a super-block T is staged in two parts, copies 0-3 after the barrier of slice
  // 4T - 6 and 4-6 after that of slice 4T - 5 (its stage was last read in slice 4T - 7); chunk_of(j)
  // is the part slice j issues (-1: none), chunk_copies(j) its number of copies.
  auto chunk_target = [&](int j) { return (j >> 2) + 2; };
  auto chunk_of = [&](int j) {
    const int q = j & 3;
    if (j < kb0 || q < 2 || chunk_target(j) >= sb_end) return -1;
    return q - 2;
  };
  auto chunk_copies = [&](int j) { const int c = chunk_of(j); return c < 0 ? 0 : c == 0 ? 4 : 3; };

  const uint32_t xs_base = (uint32_t)(uintptr_t)xs_l;
  const uint32_t row_base = (uint32_t)(uintptr_t)ws_l + (uint32_t)(wave * 32 * kQ6Win + 32 * ln);
  const uint32_t sw = xswz((uint32_t)ln);
  uint32_t a_rel[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    const uint32_t kc = 4u * (uint32_t)(s >> 1) + 2u * (uint32_t)g + (uint32_t)(s & 1);
    a_rel[s] = (uint32_t)ln * 128u + 16u * (kc ^ sw);
  }
  auto read_group = [&](uint32_t xb, int G, u32x4 (&r)[8]) {
    read_frags(xb + a_rel[G], r, std::make_integer_sequence<int, GT>{});
  };
  // the half of slice kb: its stage row, half index and lead bytes
  auto half_row = [&](int kb) { return row_base + (uint32_t)((kb >> 2) & 1) * kQ6WStage; };
  auto half_sh = [&](int kb) { return (uint32_t)((kb >> 2) * 210) & 3u; };

  f32x16_t acc[MT];
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[i][e] = 0.0f;

  // Dequantisation pieces (this lane's row, slice parity P): 0 and 1 realign a freshly read half
  // and form the slice's scales, 2..9 build 4 codes each (bn[sp][2hh], bn[sp][2hh + 1] for
  // u = p - 2 = 2 sp + hh).
  struct DeqState {
    Q6kRaw raw;
    Q6kHalf hf;
    float ds[2], bias[2];
  };
  const uint32_t k1024 = 0x64006400u;
  auto piece = [&](int p, int P, bool fresh, uint32_t sh, DeqState& st, i32x4_t (&bn)[4]) {
    if (p == 0) {
      if (fresh) q6k_align(st.raw, sh, st.hf);
    } else if (p == 1) {
      const uint32_t sw4 = st.hf.s[P];
      const float sa = (float)(int)__builtin_amdgcn_sbfe((int)sw4, 8u * (uint32_t)g, 8u);
      const float sb = (float)(int)__builtin_amdgcn_sbfe((int)sw4, 8u * (uint32_t)(g + 2), 8u);
      st.ds[0] = st.hf.d * sa;
      st.ds[1] = st.hf.d * sb;
      st.bias[0] = -1056.0f * st.ds[0];
      st.bias[1] = -1056.0f * st.ds[1];
    } else {
      const int u = p - 2, sp = u >> 1, hh = u & 1, w = (sp & 1) * 2 + hh;
      const bool second = sp >= 2;
      const uint32_t src = second ? st.hf.qb[w] : st.hf.qa[w];
      const uint32_t hq = st.hf.h[w];
      const uint32_t nib = (P ? src >> 4 : src) & geo.m0f;
      const uint32_t hb = P ? (second ? hq >> 2 : hq) : (second ? hq << 2 : hq << 4);
      const uint32_t code = __builtin_amdgcn_bitop3_b32(hb, geo.m30, nib, 0xEA);  // (hb & 0x30..) | nib
      const uint32_t e = __builtin_amdgcn_bitop3_b32(code, geo.mff, k1024, 0xEA);
      const uint32_t o = __builtin_amdgcn_bitop3_b32(code >> 8, geo.mff, k1024, 0xEA);
      const half2_t he = __builtin_bit_cast(half2_t, e), ho = __builtin_bit_cast(half2_t, o);
      const float ds = st.ds[second], bs = st.bias[second];
      bn[sp][2 * hh] = (int)pack2<VAR>(__builtin_fmaf((float)he.x, ds, bs), __builtin_fmaf((float)ho.x, ds, bs));
      bn[sp][2 * hh + 1] = (int)pack2<VAR>(__builtin_fmaf((float)he.y, ds, bs), __builtin_fmaf((float)ho.y, ds, bs));
      pin(bn[sp]);
    }
  };

  // One slice (parity P = kb % 2), as in the Q4_K kernel: group 0's fragments were read during the
  // previous slice; group 0 issues X(kb+2) and, when slice kb+1 starts a half (P = 1), the LDS reads
  // of that half; the barrier before the last group publishes X(kb+1) and frees stage kb % 3, and
  // the slice's W part is issued after it.  The dequantisation of slice kb+1 goes between the MFMAs
  // of groups 1..3, in the last slice too (on stale bytes, never used), so that no branch splits the
  // MFMA sequence.
  DeqState st;
  auto slice = [&](int kb, auto Pc, const i32x4_t (&bc)[4], i32x4_t (&bn)[4], u32x4 (&a)[2][8]) {
    constexpr int P = decltype(Pc)::value;
    const uint32_t xb = xs_base + (uint32_t)(kb % 3) * XSTAGE;
    const int kx = min(kb + 2, kb1 - 1);
    const bool more = kb + 1 < kb1;
    const uint32_t sh = half_sh(kb + 1);
    const int ch = chunk_of(kb);
    QVX_LDS uint8_t* wdst = ws_l + (chunk_target(kb) & 1) * kQ6WStage + wave * 32 * kQ6Win;
    const uint32_t wso = (uint32_t)(chunk_target(kb) * 210) & ~3u;
#pragma unroll
    for (int G = 0; G < NG; ++G) {
      u32x4(&cur)[8] = a[G & 1];
      u32x4(&nxt)[8] = a[(G + 1) & 1];
      if (G == 1 && P == 1)
        q6k_wait(cur, st.raw);
      else
        lds_wait<GT>(cur);
      if (G == NG - 1) {
        if (more) {
          // X(kb+1) landed; younger copies that may fly: the previous slice's W part (issued after
          // its barrier, so after X(kb+1)) and X(kb+2) of group 0
          const int young = chunk_copies(kb - 1);
          if (young == 4)
            wait_vm<4 + XI>();
          else if (young == 3)
            wait_vm<3 + XI>();
          else
            wait_vm<XI>();
          __builtin_amdgcn_s_barrier();
          if (ch == 0) {
#pragma unroll
            for (int c = 0; c < 4; ++c) q6k_copy(wr, wdst, voff, wso, c);
          } else if (ch == 1) {
#pragma unroll
            for (int c = 4; c < 7; ++c) q6k_copy(wr, wdst, voff, wso, c);
          }
          read_group(xs_base + (uint32_t)((kb + 1) % 3) * XSTAGE, 0, nxt);
        }
      } else {
        read_group(xb, G + 1, nxt);
      }
      if (G == 0 && P == 1) q6k_issue(half_row(kb + 1), ((kb + 1) >> 1) & 1, g, st.raw);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int t = 0; t < GT; ++t) {
        acc[t] = mfma32<VAR>(__builtin_bit_cast(i32x4_t, cur[t]), bc[G], acc[t]);
        if (G == 0 && t < XI) issue_x1(kx, t);
        if (G > 0) {
          const int slot = GT * (G - 1) + t;
#pragma unroll
          for (int p = 0; p < NP; ++p)
            if (p * NS / NP == slot) piece(p, 1 - P, P == 1, sh, st, bn);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  };

  // prologue: super-block kb0/4 and X(kb0) staged, then the next super-block and X(kb0+1) issued
  issue_w(kb0 >> 2);
  issue_x(kb0);
  wait_vm<0>();
  __builtin_amdgcn_s_barrier();
  if ((kb0 >> 2) + 1 < sb_end) issue_w((kb0 >> 2) + 1);
  issue_x(min(kb0 + 1, kb1 - 1));

  u32x4 a[2][8];
  read_group(xs_base + (uint32_t)(kb0 % 3) * XSTAGE, 0, a[0]);
  i32x4_t b0[4], b1[4];
  {
    q6k_issue(half_row(kb0), 0, g, st.raw);
    q6k_wait(st.raw);
    const uint32_t sh = half_sh(kb0);
#pragma unroll
    for (int p = 0; p < NP; ++p) piece(p, 0, true, sh, st, b0);
  }

  int kb = kb0;
  for (; kb + 1 < kb1; kb += 2) {
    slice(kb, std::integral_constant<int, 0>{}, b0, b1, a);
    slice(kb + 1, std::integral_constant<int, 1>{}, b1, b0, a);
  }
  if (kb < kb1) slice(kb, std::integral_constant<int, 0>{}, b0, b1, a);
  wait_vm<0>();

  if (gridDim.z > 1) {
    float v[MT * 16];
#pragma unroll
    for (int i = 0; i < MT * 16; ++i) v[i] = acc[i >> 4][i & 15];
    if (!split_k_last<MT * 16, 512>(v, geo.part + (size_t)tile_id * gridDim.z * (MT * 16 * 512), geo.cnt + tile_id,
                                    (int)gridDim.z, (int)blockIdx.z, tid, reinterpret_cast<int*>(xs)))
      return;
#pragma unroll
    for (int i = 0; i < MT * 16; ++i) acc[i >> 4][i & 15] = v[i];
  }

#pragma unroll
  for (int i = 0; i < MT; ++i) {
    const int n = n0 + 32 * wave + ln;
    if (n >= N) continue;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int m = m0 + 32 * i + 8 * (e >> 2) + 4 * g + (e & 3);
      if (m < M) Y[(size_t)m * N + n] = acc[i][e];
    }
  }
}

// ---- int8 variant --------------------------------------------------------------------------------
// X is quantised per 32 values to int8 (scale sx = amax/127, the public quantiser's arithmetic) by a
// prepass; the weight nibbles are int8 operands as they are.  Per 32-element block b (one Q4_K
// sub-block) one v_mfma_i32_32x32x32_i8 gives the exact integer dot I = sum q * n, folded as
//   out += sx * (ds * I - dm * qsum) = I * (sx * ds) - (sx * qsum) * dm
// (ds = d*sc, dm = dmin*m of the sub-block).  The fold is 4 VALU per output per block, against one
// MFMA per 1024 outputs: this variant is bound by the fold, not by the matrix cores.
//
// Workgroup = 256 threads, tile 128 tokens x 256 weight rows; wave w owns rows 64w..64w+63 and all
// 128 tokens (fp32 accumulators in VGPRs, as the fold updates them).  Per 64-column slice: int8 X
// (128 x 64 bytes), the tile's scales (4 x 128 floats: sx of both blocks, sx*qsum of both) and the
// weight headers + group-c quant bytes are copied into LDS (two stages, one slice ahead).
constexpr int kI8BM = 128;

// Quantiser prepass: one thread per 32-value block of the (tile-padded) M x K activations.  Writes
// q int8 [M, K] and, for slice kb and token tile t, SC[((kb * ntile + t) * 4 + a) * 128 + m % 128]
// with a = 0, 1: scale of block 2kb + a; a = 2, 3: scale * qsum of block 2kb + a - 2 (zeros for
// padding rows).  The same launch zeroes z4[0, nz4) (the tile counters of a K-split GEMM).
__global__ __launch_bounds__(256) void k_quant_q8_gemm(const uint16_t* __restrict__ X, int M, int K, int Mpad,
                                                       int8_t* __restrict__ q, float* __restrict__ sc,
                                                       float4* __restrict__ z4, size_t nz4) {
  const int nb = K / 32;
  const size_t blk = (size_t)blockIdx.x * 256 + threadIdx.x;
  for (size_t k = blk; k < nz4; k += (size_t)gridDim.x * 256) z4[k] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  if (blk >= (size_t)Mpad * nb) return;
  const int m = (int)(blk / nb), j = (int)(blk % nb);
  const int kb = j >> 1, h = j & 1, ntile = Mpad / kI8BM;
  float* base = sc + ((size_t)kb * ntile + m / kI8BM) * 4 * kI8BM + (m % kI8BM);
  if (m >= M) {
    base[h * kI8BM] = 0.0f;
    base[(2 + h) * kI8BM] = 0.0f;
    return;
  }
  const uint16_t* x = X + (size_t)m * K + 32 * j;
  float v[32];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint4 u = reinterpret_cast<const uint4*>(x)[i];
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      v[8 * i + 2 * k] = f16lo(w[k]);
      v[8 * i + 2 * k + 1] = f16hi(w[k]);
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
    for (int k = 0; k < 4; ++k) {
      float r = roundf(v[4 * i + k] * inv);
      r = fminf(fmaxf(r, -127.0f), 127.0f);
      const int qi = (int)r;
      sum += qi;
      word |= ((uint32_t)(qi & 0xFF)) << (8 * k);
    }
    packed[i] = word;
  }
  uint4* dst = reinterpret_cast<uint4*>(q + (size_t)m * K + 32 * j);
  dst[0] = make_uint4(packed[0], packed[1], packed[2], packed[3]);
  dst[1] = make_uint4(packed[4], packed[5], packed[6], packed[7]);
  base[h * kI8BM] = s;
  base[(2 + h) * kI8BM] = s * (float)sum;
}

namespace gemm {
typedef int i32x16_t __attribute__((ext_vector_type(16)));
// 32-byte rows (one Q4_K group of quant bytes): chunk g of row r at slot g ^ qswz1(r).
__device__ inline uint32_t qswz1(uint32_t r) { return ((r >> 2) ^ (r >> 3)) & 1u; }
}  // namespace gemm

__global__ __launch_bounds__(256) void k_qgemm_q4k_i8(const uint8_t* __restrict__ W, const int8_t* __restrict__ Q,
                                                      const float* __restrict__ SC, float* __restrict__ Y,
                                                      GemmGeo geo) {
  constexpr int BM = kI8BM, MT = BM / 32;
  constexpr int XS = BM * 64;          // int8 X slice
  constexpr int SS = 4 * BM * 4;       // scales of a slice
  constexpr int WST = kBN * 48;        // headers (4 KB) + group quant bytes (8 KB)
  __shared__ __attribute__((aligned(1024))) uint8_t xs[2 * XS];
  __shared__ __attribute__((aligned(1024))) uint8_t ss[2 * SS];
  __shared__ __attribute__((aligned(1024))) uint8_t ws[2 * WST];

  const int M = geo.M, N = geo.N, K = geo.K;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int ln = lane & 31, g = lane >> 5;
  const int n0 = blockIdx.x * kBN, tile = blockIdx.y, m0 = tile * BM, ntile = gridDim.y;
  const int nsl = K / 64;
  const int kb0 = blockIdx.z * geo.per_split;
  const int kb1 = min(nsl, kb0 + geo.per_split);
  if (kb0 >= kb1) return;

  const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(Q + (size_t)m0 * K), (short)0, (int)((uint32_t)min(BM, M - m0) * (uint32_t)K), (int)kRsrcWord3);
  const __amdgpu_buffer_rsrc_t sr = __builtin_amdgcn_make_buffer_rsrc(
      (void*)SC, (short)0, (int)((uint32_t)nsl * (uint32_t)ntile * (uint32_t)SS), (int)kRsrcWord3);
  const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(W + (size_t)n0 * geo.row_bytes), (short)0, (int)((uint32_t)min(kBN, N - n0) * geo.row_bytes),
      (int)kRsrcWord3);
  // X copy i (of 2) of this wave: rows 16(2w+i) + lane/4, LDS slot lane%4 of the row's 64 bytes
  // holds chunk slot ^ qswz(row).
  uint32_t xoff[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const uint32_t r = (uint32_t)(16 * (2 * wave + i) + (lane >> 2)), slot = (uint32_t)lane & 3u;
    xoff[i] = r * (uint32_t)K + 16u * (slot ^ qswz(r));
  }
  const uint32_t soff = (uint32_t)(wave * 64 + lane) * 16u;  // waves 0, 1: the two halves of the scales
  const uint32_t woff_h = (uint32_t)(64 * wave + lane) * geo.row_bytes;
  uint32_t woff_q[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const uint32_t r = (uint32_t)(64 * wave + 32 * i + (lane >> 1)), p = (uint32_t)lane & 1u;
    woff_q[i] = r * geo.row_bytes + 16u + 16u * (p ^ qswz1(r));
  }
  QVX_LDS uint8_t* xs_l = (QVX_LDS uint8_t*)xs;
  QVX_LDS uint8_t* ss_l = (QVX_LDS uint8_t*)ss;
  QVX_LDS uint8_t* ws_l = (QVX_LDS uint8_t*)ws;
  auto issue = [&](int kb) {
    const int st = kb & 1;
#pragma unroll
    for (int i = 0; i < 2; ++i)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(xr, xs_l + st * XS + (2 * wave + i) * 1024, 16, xoff[i],
                                               (uint32_t)kb * 64u, 0, 0);
    if (wave < 2)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(sr, ss_l + st * SS + wave * 1024, 16, soff,
                                               (uint32_t)(kb * ntile + tile) * (uint32_t)SS, 0, 0);
    const uint32_t sbo = (uint32_t)(kb >> 2) * 144u;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(wr, ws_l + st * WST + wave * 1024, 16, woff_h, sbo, 0, 0);
#pragma unroll
    for (int i = 0; i < 2; ++i)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(wr, ws_l + st * WST + 4096 + (2 * wave + i) * 1024, 16, woff_q[i],
                                               sbo + 32u * (uint32_t)(kb & 3), 0, 0);
  };

  const uint32_t xs_base = (uint32_t)(uintptr_t)xs_l, ss_base = (uint32_t)(uintptr_t)ss_l,
                 ws_base = (uint32_t)(uintptr_t)ws_l;
  // A: row 32i + ln, chunk 2h + g.  B rows r_j = 64w + 32j + ln.
  uint32_t a_rel[2];
  const uint32_t sw = qswz((uint32_t)ln);  // qswz(32i + ln) == qswz(ln)
#pragma unroll
  for (int h = 0; h < 2; ++h) a_rel[h] = 64u * (uint32_t)ln + 16u * ((2u * h + (uint32_t)g) ^ sw);
  uint32_t h_rel[2], q_rel[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const uint32_t r = (uint32_t)(64 * wave + 32 * j + ln);
    h_rel[j] = 16u * r;
    q_rel[j] = 4096u + 32u * r + 16u * ((uint32_t)g ^ qswz1(r));
  }
  const uint32_t s_rel = 4u * (uint32_t)(4 * g);  // token 8q + 4g + t of a 32-token tile

  float acc[MT][2][16];
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

  issue(kb0);
  wait_vm<0>();
  __builtin_amdgcn_s_barrier();
  for (int kb = kb0; kb < kb1; ++kb) {
    if (kb + 1 < kb1) issue(kb + 1);  // stage (kb+1)&1 held slice kb-1: every wave is past it
    const int st = kb & 1, c = kb & 3;
    const uint32_t xb = xs_base + (uint32_t)st * XS, sb = ss_base + (uint32_t)st * SS,
                   wb = ws_base + (uint32_t)st * WST;
    u32x4 wv[4] = {lds_read16(wb + h_rel[0]), lds_read16(wb + q_rel[0]), lds_read16(wb + h_rel[1]),
                   lds_read16(wb + q_rel[1])};
    lds_wait<4>(wv);
    const ScaleSel sel = scale_sel(c);
    float ds[2][2], dm[2][2];  // [h][j]
    i32x4_t bq[2][2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const u32x4 hd = wv[2 * j], qq = wv[2 * j + 1];
      const uint32_t scp = ((hd.y >> sel.sa) & sel.ma) | ((hd.w >> sel.sb) & sel.mb);
      const uint32_t mp = ((hd.z >> sel.sa) & sel.ma) | ((hd.w >> (sel.sb + 4u)) & sel.mb);
      const float d = f16lo(hd.x), dmin = f16hi(hd.x);
      ds[0][j] = d * ub(scp, 0);
      ds[1][j] = d * ub(scp, 1);
      dm[0][j] = dmin * ub(mp, 0);
      dm[1][j] = dmin * ub(mp, 1);
      bq[0][j] = i32x4_t{(int)(qq.x & geo.mask_lo), (int)(qq.y & geo.mask_lo), (int)(qq.z & geo.mask_lo),
                         (int)(qq.w & geo.mask_lo)};
      bq[1][j] = i32x4_t{(int)((qq.x >> 4) & geo.mask_lo), (int)((qq.y >> 4) & geo.mask_lo),
                         (int)((qq.z >> 4) & geo.mask_lo), (int)((qq.w >> 4) & geo.mask_lo)};
    }
#pragma unroll
    for (int h = 0; h < 2; ++h) {
#pragma unroll
      for (int i = 0; i < MT; ++i) {
        u32x4 av[1] = {lds_read16(xb + a_rel[h] + 2048u * i)};
        u32x4 sv[8];
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4) {
          sv[q4] = lds_read16(sb + 4u * (uint32_t)(h * BM + 32 * i + 8 * q4) + s_rel);
          sv[4 + q4] = lds_read16(sb + 4u * (uint32_t)((2 + h) * BM + 32 * i + 8 * q4) + s_rel);
        }
        lds_wait8_1(sv, av);
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const i32x16_t I = __builtin_amdgcn_mfma_i32_32x32x32_i8(__builtin_bit_cast(i32x4_t, av[0]), bq[h][j],
                                                                   i32x16_t{}, 0, 0, 0);
#pragma unroll
          for (int e = 0; e < 16; ++e) {
            const float sx = __uint_as_float(sv[e >> 2][e & 3]), sq = __uint_as_float(sv[4 + (e >> 2)][e & 3]);
            acc[i][j][e] = __builtin_fmaf((float)I[e], sx * ds[h][j], __builtin_fmaf(-sq, dm[h][j], acc[i][j][e]));
          }
        }
      }
    }
    wait_vm<0>();
    __builtin_amdgcn_s_waitcnt(0xC07F);
    __builtin_amdgcn_s_barrier();
  }

  if (gridDim.z > 1) {
    const int t = (int)(blockIdx.y * gridDim.x + blockIdx.x);
    float v[MT * 32];
#pragma unroll
    for (int a = 0; a < MT * 32; ++a) v[a] = acc[a >> 5][(a >> 4) & 1][a & 15];
    if (!split_k_last<MT * 32, 256>(v, geo.part + (size_t)t * gridDim.z * (MT * 32 * 256), geo.cnt + t,
                                    (int)gridDim.z, (int)blockIdx.z, tid, reinterpret_cast<int*>(xs)))
      return;
#pragma unroll
    for (int a = 0; a < MT * 32; ++a) acc[a >> 5][(a >> 4) & 1][a & 15] = v[a];
  }

#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int n = n0 + 64 * wave + 32 * j + ln;
      if (n >= N) continue;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int m = m0 + 32 * i + 8 * (e >> 2) + 4 * g + (e & 3);
        if (m < M) Y[(size_t)m * N + n] = acc[i][j][e];
      }
    }
}

// fp16 -> bf16 (round to nearest even), 8 values a thread; the same launch also zeroes z4[0, nz4)
// (the tile counters of a K-split GEMM) with a grid-stride loop.
__global__ __launch_bounds__(256) void k_f16_to_bf16(const uint4* __restrict__ x, uint4* __restrict__ y, size_t n8,
                                                     float4* __restrict__ z4, size_t nz4) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  for (size_t k = i; k < nz4; k += (size_t)gridDim.x * 256) z4[k] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  if (i >= n8) return;
  const uint4 v = x[i];
  y[i] = make_uint4(pack2<VAR_BF16>(f16lo(v.x), f16hi(v.x)), pack2<VAR_BF16>(f16lo(v.y), f16hi(v.y)),
                    pack2<VAR_BF16>(f16lo(v.z), f16hi(v.z)), pack2<VAR_BF16>(f16lo(v.w), f16hi(v.w)));
}

// Zero fill: four floats a thread from the first 16-byte boundary, single floats before it and in
// the tail.
__global__ __launch_bounds__(256) void k_zero_f32(float* __restrict__ p, size_t head, size_t n4, size_t n) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n4) reinterpret_cast<float4*>(p + head)[i] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  if (i < head) p[i] = 0.0f;
  const size_t t = head + 4 * n4 + i;
  if (t < n && i < 4) p[t] = 0.0f;
}

namespace {

// One stream-ordered memory pool per device for the GEMM temporaries, created on first use and
// kept for the life of the process; freed blocks stay in the pool for the next call.
std::mutex g_pool_mu;
hipMemPool_t g_pool[64];

hipMemPool_t device_pool() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return nullptr;
  std::lock_guard<std::mutex> lk(g_pool_mu);
  if (!g_pool[dev]) {
    hipMemPoolProps props{};
    props.allocType = hipMemAllocationTypePinned;
    props.location.type = hipMemLocationTypeDevice;
    props.location.id = dev;
    hipMemPool_t p = nullptr;
    if (hipMemPoolCreate(&p, &props) != hipSuccess) return nullptr;
    uint64_t keep = ~0ull;
    (void)hipMemPoolSetAttribute(p, hipMemPoolAttrReleaseThreshold, &keep);
    g_pool[dev] = p;
  }
  return g_pool[dev];
}

}  // namespace

// Zero fill by kernel (no memset nodes, so callers may capture it in a HIP graph).
void launch_zero(float* p, size_t n, hipStream_t s) {
  if (!n) return;
  const size_t mis = (reinterpret_cast<uintptr_t>(p) >> 2) & 3u;  // p is 4-byte aligned
  const size_t head = std::min(n, mis ? 4 - mis : (size_t)0), n4 = (n - head) / 4;
  const size_t threads = std::max<size_t>(n4, 4);
  k_zero_f32<<<(unsigned)((threads + 255) / 256), 256, 0, s>>>(p, head, n4, n);
}

namespace {

// One cached temporary per stream on top of the pool.  A pool allocation after a pool free on the
// same stream left the device idle ~6 us between consecutive calls on MI355X (the runtime orders the
// block's reuse behind the free); a stream's cached block needs no ordering beyond the stream's own,
// since every call that used it was issued to that stream earlier.  Streams are told apart by their
// handle (hipStreamGetId would do better, but it is newer than the HIP runtime torch bundles, which
// then refuses to load this library); a handle that hipStreamDestroy released can name a new stream,
// so a caller destroying a stream must first let the qvx calls it issued finish (include/qvx.h
// states the rule).  A block is taken only while
// idle (a second host thread on the same stream meanwhile gets a pool block), never under graph
// capture (a captured graph would then name a block that later eager calls reuse), and grows by a
// stream-ordered free and a new pool block.  Cached blocks stay until the process ends.
struct TempSlot {
  int dev = -1;
  unsigned long long sid = 0;
  void* p = nullptr;
  size_t n = 0;
  bool busy = false;
};
constexpr int kTempSlots = 32;
std::mutex g_slot_mu;
TempSlot g_slot[kTempSlots];

bool stream_key(hipStream_t s, int& dev, unsigned long long& sid) {
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  sid = (unsigned long long)(uintptr_t)s;
  if (hipGetDevice(&dev) != hipSuccess || hipStreamIsCapturing(s, &cs) != hipSuccess ||
      cs != hipStreamCaptureStatusNone) {
    (void)hipGetLastError();
    return false;
  }
  return true;
}

}  // namespace

// Stream-ordered temporary from the library's pool (nullptr on failure) and its release.
void* gemm_temp_alloc(size_t bytes, hipStream_t s) {
  hipMemPool_t pool = device_pool();
  if (!pool) return nullptr;
  int dev = 0;
  unsigned long long sid = 0;
  if (bytes && stream_key(s, dev, sid)) {
    std::lock_guard<std::mutex> lk(g_slot_mu);
    TempSlot* slot = nullptr;
    for (auto& t : g_slot)
      if (t.p && t.dev == dev && t.sid == sid) slot = &t;
    if (!slot)
      for (auto& t : g_slot)
        if (!t.p) {
          slot = &t;
          break;
        }
    if (slot && !slot->busy) {
      if (slot->p && slot->n < bytes) {
        (void)hipFreeAsync(slot->p, s);
        slot->p = nullptr;
      }
      if (!slot->p) {
        const size_t n = (bytes + ((size_t)1 << 20) - 1) & ~(((size_t)1 << 20) - 1);  // whole MiB
        void* p = nullptr;
        if (hipMallocFromPoolAsync(&p, n, pool, s) != hipSuccess) {
          (void)hipGetLastError();
          return nullptr;
        }
        *slot = TempSlot{dev, sid, p, n, false};
      }
      slot->busy = true;
      return slot->p;
    }
  }
  void* p = nullptr;
  if (hipMallocFromPoolAsync(&p, bytes, pool, s) != hipSuccess) return nullptr;
  return p;
}
void gemm_temp_free(void* p, hipStream_t s) {
  if (!p) return;
  {
    std::lock_guard<std::mutex> lk(g_slot_mu);
    for (auto& t : g_slot)
      if (t.p == p && t.busy) {
        t.busy = false;
        return;
      }
  }
  (void)hipFreeAsync(p, s);
}

namespace {
// One block of K-split tile counters per stream: made from the pool and cleared by a fill kernel in
// stream order the first time the stream needs counters (or more of them), then kept for the life
// of the process.  The GEMM kernels leave every counter they use at zero (split_k_last counts with a
// wrapping increment), and launches on one stream run one after another, so the block is zero
// whenever a launch on its stream starts and the calls need no clearing launch of their own.
struct CntSlot {
  int dev = -1;
  unsigned long long sid = 0;
  void* p = nullptr;
  size_t n = 0;
};
CntSlot g_cnt_slot[kTempSlots];
}  // namespace

// At least n zeroed tile counters that the call's launches leave zero: the stream's block, or
// nullptr under graph capture (a captured graph would then name a block that later eager calls use)
// or when none can be had; the caller then clears counters in its own temporary.
uint32_t* gemm_stream_counters(size_t n, hipStream_t s) {
  hipMemPool_t pool = device_pool();
  int dev = 0;
  unsigned long long sid = 0;
  if (!pool || !n || !stream_key(s, dev, sid)) return nullptr;
  std::lock_guard<std::mutex> lk(g_slot_mu);
  CntSlot* slot = nullptr;
  for (auto& t : g_cnt_slot)
    if (t.p && t.dev == dev && t.sid == sid) slot = &t;
  if (!slot)
    for (auto& t : g_cnt_slot)
      if (!t.p) {
        slot = &t;
        break;
      }
  if (!slot) return nullptr;
  if (slot->n < n) {
    if (slot->p) (void)hipFreeAsync(slot->p, s);
    *slot = CntSlot{};
    const size_t m = std::max<size_t>(n, 16384);
    void* p = nullptr;
    if (hipMallocFromPoolAsync(&p, m * 4, pool, s) != hipSuccess) {
      (void)hipGetLastError();
      return nullptr;
    }
    launch_zero(static_cast<float*>(p), m, s);
    *slot = CntSlot{dev, sid, p, m};
  }
  return static_cast<uint32_t*>(slot->p);
}

// ---- per-32 Q8 activation quantiser --------------------------------------------------------------
// One thread per block of 32 values; fp32 math as the oracle states it.
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

namespace {

// Whole super-blocks of K per split, and the split count that results.
inline int split_per(int nsl, int splits) { return ((nsl + splits - 1) / splits + 3) & ~3; }

// One launch of the Q4_K GEMM: BM tokens a tile, K splits, the 1-D tile numbering.
struct Q4kLaunch {
  int bm, splits, ntiles;
  TileMap tm;
};
struct Q4kPlan {
  int n;
  Q4kLaunch l[2];
};

template <int VAR, int BM>
bool launch_q4k(float* out, const void* w, const uint16_t* X, int M, int N, int K, const Q4kLaunch& L,
                float* part, uint32_t* cnt, hipStream_t s) {
  static LdsLimit lim;
  if (!lds_ready(reinterpret_cast<const void*>(&k_qgemm_q4k<VAR, BM>), lim, 0)) return false;
  if (L.splits > 1 && (!part || !cnt)) return false;
  const int per = split_per(K / 64, L.splits);
  GemmGeo geo{M, N, K, (uint32_t)(K / 256) * 144u, per, 0x0F0F0F0Fu, 0xF0F0F0F0u, 0x000F000Fu, 0x00F000F0u, part, cnt};
  k_qgemm_q4k<VAR, BM><<<dim3(L.ntiles, 1, L.splits), 512, 0, s>>>(static_cast<const uint8_t*>(w), X, out, geo, L.tm);
  return true;
}

template <int VAR, int BM>
bool launch_q4kq(float* out, const void* w, const uint16_t* X, int M, int N, int K, const Q4kLaunch& L,
                 hipStream_t s) {
  static LdsLimit lim;
  if (!lds_ready(reinterpret_cast<const void*>(&k_qgemm_q4kq<VAR, BM>), lim, 0)) return false;
  if (L.bm != BM || L.splits != 1) return false;
  GemmGeo geo{M, N, K, (uint32_t)(K / 256) * 144u, K / 64, 0x0F0F0F0Fu, 0xF0F0F0F0u, 0x000F000Fu, 0x00F000F0u,
              nullptr, nullptr};
  k_qgemm_q4kq<VAR, BM><<<dim3(L.ntiles), 256, 0, s>>>(static_cast<const uint8_t*>(w), X, out, geo, L.tm);
  return true;
}

}  // namespace

// Compute units of the current device (cached per device).
int device_cus() {
  static std::atomic<int> cache[kMaxDevices] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return 256;
  int n = cache[dev].load(std::memory_order_relaxed);
  if (n <= 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cache[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

namespace {

inline int cdiv(int a, int b) { return (a + b - 1) / b; }

// Tile plan for an M x N x K launch on `cus` compute units (one 512-thread workgroup fits a CU).
//  * Grids smaller than the chip: 128-token tiles, splitting K (each split stores its partial tile;
//    the last split of a tile sums them in split order) only while the grid is below ~200
//    workgroups.
//  * Otherwise the cheapest of: a uniform grid of 256-, 192- or 128-token tiles, or two launches,
//    the first of 256-token tiles from token 0 and the second of 192- or 128-token tiles for the
//    rest, with two kinds of columns (x columns with a1 + b1 tiles, the others with a2 + b2).  The
//    cost of a launch is its rounds of workgroups times the tile time, BM / 256 plus a fixed part
//    for the prologue and the output store.  For 2048 x 14336 on 256 CUs this gives 256 tiles of
//    256 tokens (48 columns x 5 + 8 x 2) and 256 tiles of 192 (48 x 4 + 8 x 8): 1.75 rounds of
//    256-token tile time where a uniform grid takes 2.
void q4k_plan(int M, int N, int K, int cus, Q4kPlan& p) {
  const int nt = cdiv(N, kBN), nsl = K / 64;
  auto uniform = [&](int bm, int splits) {
    Q4kLaunch L{bm, splits, nt * cdiv(M, bm), TileMap{nt, cdiv(M, bm), 0, 1, 0}};
    return L;
  };
  p.n = 1;
  if (nt * cdiv(M, 256) < 224 * cus / 256) {
    int splits = 1;
    const int tiles = nt * cdiv(M, 128);
    while (tiles * splits < 200 * cus / 256 && nsl / (splits * 2) >= 8) splits *= 2;
    const int per = split_per(nsl, splits);
    p.l[0] = uniform(128, (nsl + per - 1) / per);
    return;
  }
  auto cost = [&](int bm, int tiles) { return tiles ? cdiv(tiles, cus) * (bm / 256.0 + 0.05) : 0.0; };
  double best = cost(256, nt * cdiv(M, 256));
  p.l[0] = uniform(256, 1);
  for (int bm : {192, 128}) {
    const double c = cost(bm, nt * cdiv(M, bm));
    if (c < best - 1e-9) {
      best = c;
      p.l[0] = uniform(bm, 1);
    }
  }
  const int A = cdiv(M, 256);
  for (int bmb : {192, 128})
    for (int a1 = std::max(1, A - 8); a1 <= A; ++a1)
      for (int a2 = std::max(0, A - 8); a2 <= a1; ++a2) {
        const int b1 = M > 256 * a1 ? cdiv(M - 256 * a1, bmb) : 0;
        const int b2 = M > 256 * a2 ? cdiv(M - 256 * a2, bmb) : 0;
        for (int x = 1; x <= nt; ++x) {
          const int ta = x * a1 + (nt - x) * a2, tb = x * b1 + (nt - x) * b2;
          if (!tb) continue;
          const double c = cost(256, ta) + cost(bmb, tb) + 0.02;
          if (c < best - 1e-9) {
            best = c;
            p.n = 2;
            p.l[0] = Q4kLaunch{256, 1, ta, TileMap{x, a1, 0, a2, 0}};
            p.l[1] = Q4kLaunch{bmb, 1, tb, TileMap{x, b1, 256 * a1, b2, 256 * a2}};
          }
        }
      }
}

// 256-token tiles run on the 4-wave kernel (k_qgemm_q4kq; measured 3-9 % faster than the 8-wave
// kernel's 256-token tiles on MI355X at M = 1024-4096, N = 14336 and 28672), the others on the
// 8-wave kernel.  Only 128-token launches split K.
template <int VAR>
bool launch_one(float* out, const void* w, const uint16_t* X, int M, int N, int K, const Q4kLaunch& L,
                float* part, uint32_t* cnt, hipStream_t s) {
  switch (L.bm) {
    case 256: return launch_q4kq<VAR, 256>(out, w, X, M, N, K, L, s);
    case 192: return launch_q4k<VAR, 192>(out, w, X, M, N, K, L, part, cnt, s);
    case 128: return launch_q4k<VAR, 128>(out, w, X, M, N, K, L, part, cnt, s);
    default: return false;
  }
}

// Workspace of a K-split plan (partial tiles, then the tile counters, 256-byte aligned); 0 when
// the plan does not split K (two-launch plans never do).
size_t q4k_split_bytes(const Q4kPlan& p) {
  const Q4kLaunch& L = p.l[0];
  if (L.splits <= 1) return 0;
  const size_t parts = (size_t)L.ntiles * L.splits * L.bm * kBN * 4;
  return parts + (((size_t)L.ntiles * 4 + 255) & ~(size_t)255);
}

// The Q6_K kernel (k_qgemm_q6k8): 128-token tiles, K split while the grid is below ~200 workgroups
// and each split keeps >= 16 slices (its prologue stages two super-blocks; measured against >= 8
// and >= 32 on the Llama-3-8B shapes: 4-7 % faster than >= 8 below M = 384, up to 23 % at 384).
void q6k8_plan(int M, int N, int K, int cus, Q4kPlan& p) {
  const int nt = cdiv(N, kBN), nsl = K / 64, tiles = nt * cdiv(M, 128);
  int splits = 1;
  while (tiles * splits < 200 * cus / 256 && nsl / (splits * 2) >= 16) splits *= 2;
  const int per = split_per(nsl, splits);
  p.n = 1;
  p.l[0] = Q4kLaunch{128, (nsl + per - 1) / per, tiles, TileMap{nt, cdiv(M, 128), 0, 1, 0}};
}

// 1 if k_qgemm_q6k8 takes this call: an even number of blocks a row (every row's blocks share one
// dword alignment), W 4-byte and X 16-byte aligned, a tile's X rows and W rows within 31-bit buffer
// offsets.
bool q6k8_supported(const void* w, const uint16_t* X, int K, int N) {
  if (K <= 0 || K % 512 != 0 || N <= 0) return false;
  if ((reinterpret_cast<uintptr_t>(w) & 3u) || (reinterpret_cast<uintptr_t>(X) & 15u)) return false;
  const size_t row_bytes = (size_t)(K / 256) * 210u;
  return (size_t)128 * (size_t)K * 2u < (1u << 31) && (size_t)kBN * row_bytes < (1u << 31);
}

// ws: the workspace of q4k_split_bytes(p) bytes; scnt: zeroed counters to use in place of the
// workspace's (a stream's block), or nullptr (the workspace's counters are then already zero).
template <int VAR>
bool launch_q6k8(float* out, const void* w, const uint16_t* X, int M, int N, int K, const Q4kPlan& p, void* ws,
                 uint32_t* scnt, hipStream_t s) {
  static LdsLimit lim;
  if (!lds_ready(reinterpret_cast<const void*>(&k_qgemm_q6k8<VAR>), lim, 0)) return false;
  const Q4kLaunch& L = p.l[0];
  const size_t sb = q4k_split_bytes(p);
  float* part = sb ? static_cast<float*>(ws) : nullptr;
  uint32_t* cnt = !sb ? nullptr
                 : scnt ? scnt
                        : reinterpret_cast<uint32_t*>(static_cast<uint8_t*>(ws) + (size_t)L.ntiles * L.splits * 128 * kBN * 4);
  if (L.splits > 1 && !ws) return false;
  Q6kGeo geo{M, N, K, (uint32_t)(K / 256) * 210u, split_per(K / 64, L.splits), 0x0F0F0F0Fu, 0x30303030u,
             0x00FF00FFu, part, cnt};
  k_qgemm_q6k8<VAR><<<dim3(L.ntiles, 1, L.splits), 512, 0, s>>>(static_cast<const uint8_t*>(w), X, out, geo, L.tm);
  return true;
}

// ws: the workspace of q4k_split_bytes(p) bytes; scnt as for launch_q6k8.
template <int VAR>
bool launch_var(float* out, const void* w, const uint16_t* X, int M, int N, int K, const Q4kPlan& p, void* ws,
                uint32_t* scnt, hipStream_t s) {
  const size_t sb = q4k_split_bytes(p);
  float* part = sb ? static_cast<float*>(ws) : nullptr;
  uint32_t* cnt = !sb ? nullptr
                 : scnt ? scnt
                        : reinterpret_cast<uint32_t*>(static_cast<uint8_t*>(ws) +
                                                      (size_t)p.l[0].ntiles * p.l[0].splits * p.l[0].bm * kBN * 4);
  for (int i = 0; i < p.n; ++i)
    if (!launch_one<VAR>(out, w, X, M, N, K, p.l[i], part, cnt, s)) return false;
  return true;
}

}  // namespace

// The Q4_K tile plan as 8 ints a launch (qvx_qgemm_plan_q4k); returns the launch count.
int q4k_plan_desc(int M, int N, int K, int cus, int* desc, int cap) {
  Q4kPlan p;
  q4k_plan(M, N, K, cus > 0 ? cus : device_cus(), p);
  for (int i = 0; i < p.n && i < cap; ++i) {
    const Q4kLaunch& L = p.l[i];
    const int v[8] = {L.bm, L.splits, L.ntiles, L.tm.cols_a, L.tm.mt_a, L.tm.base_a, L.tm.mt_b, L.tm.base_b};
    for (int j = 0; j < 8; ++j) desc[8 * i + j] = v[j];
  }
  return p.n;
}

// The prefill GEMM through a 16-bit dequantised weight and the plain MFMA GEMM (qvx_gemm16.hip);
// returns a QVX status (0 ok, -1 type, -5 HIP, -7 range).
int launch_qgemm_via16(float* out, const void* w, uint32_t t, const uint16_t* X, int M, int rows, int cols, bool bf16,
                       hipStream_t s, void* ws, size_t ws_cap);
// The dequantising MFMA GEMM of the other weight types (qvx_gemm_deq.hip).
bool qgemm_deq_supported(uint32_t t, const void* w, const uint16_t* X, int K, int N, size_t row_bytes);
size_t qgemm_deq_split_bytes(int M, int N, int K, size_t* counters);
bool launch_qgemm_deq(uint32_t t, float* out, const void* w, const uint16_t* X, int M, int N, int K, size_t row_bytes,
                      bool bf16, void* split_ws, hipStream_t s);

// Device memory for the call's temporaries: from the library's pool when ws is null, else the
// caller's region [ws, ws + ws_cap) (the no-allocation entry point's scratch; -7 when the call needs
// more).  Returns the region, or null.
static void* gemm_ws(size_t need, void* ws, size_t ws_cap, hipStream_t s) {
  if (ws) return need <= ws_cap ? ws : nullptr;
  return gemm_temp_alloc(need, s);
}
static void gemm_ws_release(void* p, void* ws, hipStream_t s) {
  if (!ws) gemm_temp_free(p, s);
}

int launch_qgemm(float* out, const void* w, uint32_t t, const uint16_t* X, int M, int rows, int cols, int variant,
                 hipStream_t s, void* ws, size_t ws_cap) {
  const int no_mem = ws ? -7 : -5;  // a caller's region too small for the call / pool allocation failed
  if (t != T_Q4_K) {
    if (variant == VAR_I8) return -1;
    const TypeInfo* ti = type_info(t);
    if (!ti) return -1;
    const size_t row_bytes = (size_t)(cols / (int)ti->block) * ti->bytes;
    // Q6_K with an even number of blocks a row: the Q4_K kernel's pipeline (k_qgemm_q6k8), except
    // for large calls that may allocate: from M = 1024 on a weight of >= 32 Mi elements the weight
    // dequantised to 16 bits and the plain GEMM are faster (measured on MI355X, ffn_down 14336 ->
    // 4096: M = 1024 / 2048 / 4096 in 163 / 263 / 449 us against 182 / 329 / 664 on k_qgemm_q6k8,
    // fp16), while the no-allocation call keeps the raw-block kernel (its scratch cannot hold the
    // 16-bit weight) ...
    if (t == T_Q6_K && !ws && M >= 1024 && (size_t)rows * (size_t)cols >= ((size_t)32 << 20))
      return launch_qgemm_via16(out, w, t, X, M, rows, cols, variant == VAR_BF16, s, ws, ws_cap);
    if (t == T_Q6_K && q6k8_supported(w, X, cols, rows)) {
      Q4kPlan plan;
      q6k8_plan(M, rows, cols, device_cus(), plan);
      const size_t n = (size_t)M * (size_t)cols;
      const size_t xbytes = variant == VAR_BF16 ? (n * 2u + 255) & ~(size_t)255 : 0;
      const size_t sbytes = q4k_split_bytes(plan);
      uint8_t* tmp = nullptr;
      if (xbytes + sbytes) {
        tmp = static_cast<uint8_t*>(gemm_ws(xbytes + sbytes, ws, ws_cap, s));
        if (!tmp) return no_mem;
      }
      // the K split's counters: the stream's zeroed block for calls that may allocate, else the
      // temporary's, cleared by the bf16 prepass or a zero kernel
      uint32_t* scnt = sbytes && !ws ? gemm_stream_counters((size_t)plan.l[0].ntiles, s) : nullptr;
      const size_t cbytes = sbytes && !scnt ? (((size_t)plan.l[0].ntiles * 4 + 255) & ~(size_t)255) : 0;
      float* cnt = cbytes ? reinterpret_cast<float*>(tmp + xbytes + sbytes - cbytes) : nullptr;
      const uint16_t* Xg = X;
      if (variant == VAR_BF16) {
        k_f16_to_bf16<<<(unsigned)((n / 8 + 255) / 256), 256, 0, s>>>(
            reinterpret_cast<const uint4*>(X), reinterpret_cast<uint4*>(tmp), n / 8, reinterpret_cast<float4*>(cnt),
            cbytes / 16);
        Xg = reinterpret_cast<const uint16_t*>(tmp);
      } else if (cbytes) {
        launch_zero(cnt, cbytes / 4, s);
      }
      void* sws = sbytes ? tmp + xbytes : nullptr;
      const bool ok = variant == VAR_BF16 ? launch_q6k8<VAR_BF16>(out, w, Xg, M, rows, cols, plan, sws, scnt, s)
                                          : launch_q6k8<VAR_F16>(out, w, Xg, M, rows, cols, plan, sws, scnt, s);
      if (tmp) gemm_ws_release(tmp, ws, s);
      return ok ? 0 : -5;
    }
    // ... the other weight types: their rows dequantised into the MFMA tiles (cols % 64 == 0, aligned
    // operands) ...
    if (qgemm_deq_supported(t, w, X, cols, rows, row_bytes)) {
      // Temporaries: the bf16 copy of X (bf16 variant), then a K split's partial tiles and tile
      // counters, the counters cleared by the bf16 prepass or a zero kernel.
      const size_t n = (size_t)M * (size_t)cols;
      const size_t xbytes = variant == VAR_BF16 ? (n * 2u + 255) & ~(size_t)255 : 0;
      size_t cbytes = 0;
      const size_t sbytes = qgemm_deq_split_bytes(M, rows, cols, &cbytes);
      uint8_t* tmp = nullptr;
      if (xbytes + sbytes) {
        tmp = static_cast<uint8_t*>(gemm_ws(xbytes + sbytes, ws, ws_cap, s));
        if (!tmp) return no_mem;
      }
      float* cnt = sbytes ? reinterpret_cast<float*>(tmp + xbytes + sbytes - cbytes) : nullptr;
      const uint16_t* Xg = X;
      if (variant == VAR_BF16) {
        k_f16_to_bf16<<<(unsigned)((n / 8 + 255) / 256), 256, 0, s>>>(
            reinterpret_cast<const uint4*>(X), reinterpret_cast<uint4*>(tmp), n / 8, reinterpret_cast<float4*>(cnt),
            cbytes / 16);
        Xg = reinterpret_cast<const uint16_t*>(tmp);
      } else if (sbytes) {
        launch_zero(cnt, cbytes / 4, s);
      }
      const bool ok = launch_qgemm_deq(t, out, w, Xg, M, rows, cols, row_bytes, variant == VAR_BF16,
                                       sbytes ? tmp + xbytes : nullptr, s);
      if (tmp) gemm_ws_release(tmp, ws, s);
      return ok ? 0 : -5;
    }
    // ... else dequantised into 16 bits per panel of rows, then the plain 16-bit MFMA GEMM
    // (qvx_gemm16.hip).
    return launch_qgemm_via16(out, w, t, X, M, rows, cols, variant == VAR_BF16, s, ws, ws_cap);
  }
  if ((reinterpret_cast<uintptr_t>(w) & 15u) || (reinterpret_cast<uintptr_t>(X) & 15u)) return -7;
  // Buffer offsets are 32-bit: a tile's rows must span less than 2 GiB.
  if ((size_t)256 * (size_t)cols * 2u >= (1u << 31) || (size_t)kBN * (size_t)(cols / 256) * 144u >= (1u << 31))
    return -7;
  if (variant == VAR_BF16 || variant == VAR_F16) {
    // Temporaries: the bf16 copy of X (bf16 variant), then a K-split plan's partial tiles and tile
    // counters.  The counters start at zero: the bf16 prepass clears them in the same launch,
    // otherwise a zero kernel does.
    Q4kPlan plan;
    q4k_plan(M, rows, cols, device_cus(), plan);
    const size_t n = (size_t)M * (size_t)cols;
    const size_t xbytes = variant == VAR_BF16 ? (n * 2u + 255) & ~(size_t)255 : 0;
    const size_t sbytes = q4k_split_bytes(plan);
    void* tmp = nullptr;
    if (xbytes + sbytes) {
      tmp = gemm_ws(xbytes + sbytes, ws, ws_cap, s);
      if (!tmp) return no_mem;
    }
    uint8_t* split_ws = static_cast<uint8_t*>(tmp) + xbytes;
    // the K split's counters: the stream's zeroed block for calls that may allocate, else the
    // temporary's, cleared by the bf16 prepass or a zero kernel
    uint32_t* scnt = sbytes && !ws ? gemm_stream_counters((size_t)plan.l[0].ntiles, s) : nullptr;
    const size_t cbytes = sbytes && !scnt ? (((size_t)plan.l[0].ntiles * 4 + 255) & ~(size_t)255) : 0;
    float* cnt = cbytes ? reinterpret_cast<float*>(split_ws + sbytes - cbytes) : nullptr;
    const size_t ncnt4 = cbytes / 16;
    const uint16_t* Xg = X;
    if (variant == VAR_BF16) {
      k_f16_to_bf16<<<(unsigned)((n / 8 + 255) / 256), 256, 0, s>>>(
          reinterpret_cast<const uint4*>(X), static_cast<uint4*>(tmp), n / 8, reinterpret_cast<float4*>(cnt), ncnt4);
      Xg = static_cast<const uint16_t*>(tmp);
    } else if (cbytes) {
      launch_zero(cnt, ncnt4 * 4, s);
    }
    const bool ok = variant == VAR_BF16 ? launch_var<VAR_BF16>(out, w, Xg, M, rows, cols, plan, split_ws, scnt, s)
                                        : launch_var<VAR_F16>(out, w, Xg, M, rows, cols, plan, split_ws, scnt, s);
    if (tmp) gemm_ws_release(tmp, ws, s);
    return ok ? 0 : -5;
  }
  if (variant == VAR_I8) {
    static LdsLimit lim;
    if (!lds_ready(reinterpret_cast<const void*>(&k_qgemm_q4k_i8), lim, 0)) return -5;
    const int ntile = (M + kI8BM - 1) / kI8BM, Mpad = ntile * kI8BM, nsl = cols / 64;
    // two int8 workgroups fit a CU (44 KB LDS, <= 256 registers): aim for ~two per CU
    const int tiles = ((rows + kBN - 1) / kBN) * ntile;
    int splits = 1;
    while (tiles * splits < 448 && nsl / (splits * 2) >= 8) splits *= 2;
    const int per = split_per(nsl, splits);
    splits = (nsl + per - 1) / per;
    // Temporaries: the Q8 copy of X, its scales, then a K split's partial tiles and tile counters
    // (cleared by the quantiser launch).
    const size_t qbytes = ((size_t)M * cols + 255) & ~(size_t)255;
    const size_t sbytes = (size_t)nsl * ntile * 4 * kI8BM * 4;
    if (sbytes >= (1u << 31)) return -7;
    const size_t pbytes = splits > 1 ? (size_t)tiles * splits * kI8BM * kBN * 4 : 0;
    const size_t cbytes = splits > 1 ? (((size_t)tiles * 4 + 255) & ~(size_t)255) : 0;
    uint8_t* qb = static_cast<uint8_t*>(gemm_ws(qbytes + sbytes + pbytes + cbytes, ws, ws_cap, s));
    if (!qb) return no_mem;
    int8_t* q = reinterpret_cast<int8_t*>(qb);
    float* sc = reinterpret_cast<float*>(qb + qbytes);
    float* part = splits > 1 ? reinterpret_cast<float*>(qb + qbytes + sbytes) : nullptr;
    uint32_t* cnt = splits > 1 ? reinterpret_cast<uint32_t*>(qb + qbytes + sbytes + pbytes) : nullptr;
    const size_t nblk = (size_t)Mpad * (cols / 32);
    k_quant_q8_gemm<<<(unsigned)((nblk + 255) / 256), 256, 0, s>>>(
        X, M, cols, Mpad, q, sc, reinterpret_cast<float4*>(cnt), cbytes / 16);
    GemmGeo geo{M, rows, cols, (uint32_t)(cols / 256) * 144u, per, 0x0F0F0F0Fu, 0xF0F0F0F0u, 0x000F000Fu,
                0x00F000F0u, part, cnt};
    dim3 grid((rows + kBN - 1) / kBN, ntile, splits);
    k_qgemm_q4k_i8<<<grid, 256, 0, s>>>(static_cast<const uint8_t*>(w), q, sc, out, geo);
    gemm_ws_release(qb, ws, s);
    return 0;
  }
  return -1;
}

}  // namespace qvx
