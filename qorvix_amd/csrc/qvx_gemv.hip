// qvx_gemv.hip -- decode GEMV (M = 1..16) over raw GGUF blocks on gfx950.
//
// out[v, r] = sum_k dequant(W)[r, k] * X[v, k]   (the reference's qmatmul / qmatmulN,
// runtime/src/qmatmul.cpp:28-115), fp32 activations in, fp32 out.
//
// Arithmetic: integer dot products on the quant codes.
//  * A row of K = cols elements is cut into S "slots" of R runs of 16 elements: R = 4 (64
//    elements: one 64-element scale group of a Q4_K super-block, or two Q4_0 / Q8_0 blocks) or
//    R = 2 (Q6_K: two quarter-runs that share a 16-element column range).
//  * Each workgroup first converts the activations of every slot to 15-bit fixed point,
//    q = rn(x / amax * 16383) with amax the slot's largest |x| (v_cvt_pknorm_i16_f32), so
//    x = q * sx + e with sx = amax / 16383 and |e| <= sx / 2 (at most 3.1e-5 of the slot's
//    largest activation).  q is split as q = 128 qh + ql with qh = q >> 7 in [-128, 127] and
//    ql = q & 127, both signed bytes, and stored in LDS with the run sums of q.
//  * Quant codes are unpacked in registers to signed bytes and multiplied with v_dot4_i32_i8
//    against qh and ql: T = sum(code q) over a run is exact in int32.  High nibbles are taken in
//    place as 16 (n - 8) (one v_bitop3: (w & 0xF0) ^ 0x80), so sum(n q) = (T + 128 Q) / 16 with
//    Q = sum(q) over the run.  The block's affine map is applied once per slot:
//      Q4_K  d*(sc_a Ta + sc_b Tb) - dmin*(m_a Qa + m_b Qb)          (sub-blocks a, b of the group)
//      Q6_K  d*(sc_a (Ta - 32 Qa) + sc_b (Tb - 32 Qb))
//      Q4_0  d*sum((n - 8) q)   Q8_0  d*sum(c q)                       (per block)
//    and each row's partial is scaled by sx once.  The only error beyond fp32 rounding is the
//    activations' fixed-point step, far inside the 1e-3 max-relative bound of the operator.
//
// Work decomposition:
//  * A workgroup has G groups of S' lanes (S' = S rounded up to a multiple of 64, or to a power of
//    two >= 8 when S < 64); lane j of a group owns slot j for the whole kernel and keeps its
//    fixed-point activations in registers.  Workgroup b owns the contiguous rows
//    [rows*b/nwg, rows*(b+1)/nwg); group g takes rows g, g+G, ... of them (n <= RMAX rows).
//  * A lane requests its activations first and then the quant bytes of all its rows, with no
//    branches between the loads, so the conversion waits only for the activations and each row's
//    arithmetic only for that row's bytes while later rows are still arriving.
//  * Each output's S' lane partials are summed with DPP / permlane swaps inside each wave (only
//    commutative adds, so every lane holds the same bits) and, for groups wider than a wave, by
//    one thread over the wave sums in wave order.  No step depends on NV, so qvx_qmatmul_n is
//    bit-identical to qvx_qmatmul per vector, the reference's promise for qmatmulN
//    (runtime/include/qorvix/runtime/qmatmul.hpp:31-32).
//
// Requirements checked by the launcher: W and X 16-byte aligned, row pitch a multiple of 16 bytes,
// K a whole number of slots, S' <= 1024.  Other shapes go to the generic kernel in qvx_dequant.hip.
#include "qvx_gemv_valu.hpp"

namespace qvx {

template <uint32_t T, int NV, int RMAX, int TPT, int PF, bool CH, bool NORM>
__global__ __launch_bounds__((gemv_threads<T, NV>())) void k_gemv(const uint8_t* __restrict__ W, const float* __restrict__ X,
                                               float* __restrict__ Y, int rows, int cols, Geo geo,
                                               const float* __restrict__ NW, float eps) {
  gemv_valu_body<T, NV, RMAX, TPT, PF, CH, NORM>(W, X, Y, rows, cols, geo, NW, eps, blockIdx.x, threadIdx.x,
                                                 threadIdx.y);
}

// ---- batched Q6_K on the matrix cores ----------------------------------------------------------
// qmatmul_n over Q6_K weights, NV (4, 8 or 16) vectors a launch, each weight byte streamed once, and
// bit-identical per vector to the one-vector VALU kernel above (k_gemv<T_Q6_K, ...>):
//  * the same slots (32 elements: quarters e and e+2 of a 16-element column range of a
//    128-element half, Lane<T_Q6_K>), the same activation conversion (convert_task<2>), the same
//    exact integer run sums -- here sum (code - 32) q over a run, which equals the VALU kernel's
//    dotq - 32 Q -- and the same float fold (Lane<T_Q6_K>::fold, times sx);
//  * the same reduction.  The VALU kernel sums a row's slot partials over 64-lane spans with DPP and
//    permlane swaps: a balanced pairwise tree over each 64 consecutive slots, then, for rows of
//    more than 64 slots, those 64-slot sums in order from 0.  Here a lane adds the two slots of a
//    pair (tree level 1); a step (one half super-block: two pairs) sums its pairs (level 2); the
//    16 steps of a 64-slot block are summed as a balanced tree (levels 3-6); the blocks in the same
//    order from 0.
// MFMA (v_mfma_i32_32x32x16_i8, one per 16-element quarter of a slot pair): A = 32 rows (vector v,
// part p: qh / ql) x the quarter's 16 fixed-point activation bytes; B = the quarter's 16 signed
// codes (code - 32) of 32 weight rows.  Lane l supplies row / column l%32 and K elements
// 8 (l/32)..+7 of both operands; its accumulator holds column l%32 (weight row) and rows
// 8j + 4 (l/32) + i (i, j = 0..3): the qh and ql sums of vectors 4j + 2 (l/32) + {0, 1}.  The run
// sum is T = (qh sum) * 128 + (ql sum), as dotq forms it.
typedef uint32_t u32x3a4_t __attribute__((ext_vector_type(3), aligned(4)));

// Raw bytes of half h of one super-block of a lane's row (l%32) for its K half g = l/32: the ql
// pieces (q&1, t) at 64h + 32(q&1) + 16t + 8g, the qh pieces t at 128 + 32h + 16t + 8g (8 bytes
// each, read as dword-aligned 12-byte windows, never past the super-block), and the super-block's
// 16 scale bytes (a 20-byte window ending at or before byte 210), d and byte misalignment.
struct Q6Half {
  u32x3a4_t ql[4], qh[2];
  uint32_t sc[5], d, sh;
};
// The code pieces of half h (ql, qh windows) and the super-block's scales, d and misalignment.
__device__ __attribute__((always_inline)) inline void q6_load_codes(const uint8_t* base, uint32_t sh, int g, int h,
                                                                    Q6Half& r) {
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int off = 64 * h + 32 * (k >> 1) + 16 * (k & 1) + 8 * g;
    r.ql[k] = *reinterpret_cast<const u32x3a4_t*>(base + off - sh);
  }
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const int off = 128 + 32 * h + 16 * k + 8 * g;
    r.qh[k] = *reinterpret_cast<const u32x3a4_t*>(base + off - sh);
  }
}
__device__ __attribute__((always_inline)) inline void q6_load_scales(const uint8_t* base, uint32_t sh, Q6Half& r) {
  r.sh = sh;
  const uint8_t* sw = base + 190 - ((sh + 2u) & 3u);  // [188, 208) or [190, 210) of the super-block
#pragma unroll
  for (int k = 0; k < 5; ++k) r.sc[k] = ldg4(sw + 4 * k);
  r.d = ldg2(base + 208);
}
// 16 signed codes (code - 32) of quarter Q (elements 8g..8g+7 of it) of pair t as two dwords.
template <int Q>
__device__ __attribute__((always_inline)) inline void q6_codes(const Q6Half& r, int t, uint32_t (&c)[2]) {
  const u32x3a4_t& l = r.ql[2 * (Q & 1) + t];
  const u32x3a4_t& hh = r.qh[t];
  const uint32_t ql[2] = {align_bytes(l.y, l.x, r.sh), align_bytes(l.z, l.y, r.sh)};
  const uint32_t qh[2] = {align_bytes(hh.y, hh.x, r.sh), align_bytes(hh.z, hh.y, r.sh)};
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const uint32_t lo = (Q >> 1) ? (ql[i] >> 4) : ql[i];
    const uint32_t hi = Q == 0 ? qh[i] << 4 : Q == 1 ? qh[i] << 2 : Q == 2 ? qh[i] : qh[i] >> 2;  // bits 2Q, 2Q+1 -> 4, 5
    const uint32_t u = (lo & 0x0F0F0F0Fu) | (hi & 0x30303030u) | 0x80808080u;                  // code + 128 per byte
    c[i] = (u - 0x20202020u) ^ 0x80808080u;                                                    // code - 32
  }
}

// A lane's activation operands of one slot pair: its four A fragments (quarter q = e + 2 run: vector
// av = l%32 / 2, part ap = l%2 (qh / ql), elements 8g..8g+7 of the run; lanes past the launch's NV
// vectors hold zeros) and the steps sx of the NV/2 vectors v = 4j + 2g + b its accumulators hold.
template <int NV>
struct Q6Act {
  uint64_t a[4];
  float sx[2][NV / 2];
};
// Reads a pair's operands from its converted-activation records (record (v, e) at word v*vstride +
// 20 e, the convert_task<2> layout) and compact steps (sx of (e, g, 2j + b) at e*NV + g*NV/2 + 2j + b),
// in LDS or in global memory.
template <int NV>
__device__ __attribute__((always_inline)) inline void q6_act_load(const uint32_t* xrec, int vstride, const float* sxc,
                                                                  int lane, Q6Act<NV>& x) {
  const int ln = lane & 31, g = lane >> 5, av = ln >> 1, ap = ln & 1;
#pragma unroll
  for (int e = 0; e < 2; ++e)
#pragma unroll
    for (int k = 0; k < NV / 2; ++k) x.sx[e][k] = sxc[e * NV + g * (NV / 2) + k];
#pragma unroll
  for (int q = 0; q < 4; ++q)
    x.a[q] = av < NV ? *reinterpret_cast<const uint64_t*>(xrec + av * vstride + (q & 1) * 20 + ap * 8 + 4 * (q >> 1) + 2 * g)
                     : 0ull;
}

// One slot pair (h, t) of a super-block half r for this lane's row (l%32): each vector's pair sum
// p(slot 2p) + p(slot 2p+1), for the 8 (NV = 16), 4 (NV = 8) or 2 (NV = 4) vectors v = 4j + 2g + b
// this lane's accumulators hold.
template <int NV>
__device__ __attribute__((always_inline)) inline void q6_pair_fold(const Q6Half& r, int h, int t, const Q6Act<NV>& x,
                                                                   int lane, float (&P)[NV / 2]) {
  using L6 = Lane<T_Q6_K>;
  constexpr int NJ = NV / 4;
  const float keep = 1.0f;
  // 6-bit scales of slots e = 0, 1: sc[8h + t + 2e] and sc[8h + t + 2e + 4]
  uint32_t s4[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) s4[i] = r.sh ? align_bytes(r.sc[i + 1], r.sc[i], 2u) : r.sc[i + 1];
  const float d = f16lo(r.d);
  float p0[NV / 2];
#pragma unroll
  for (int e = 0; e < 2; ++e) {
    uint32_t ca[2], cb[2];
    if (e == 0) {
      q6_codes<0>(r, t, ca);
      q6_codes<2>(r, t, cb);
    } else {
      q6_codes<1>(r, t, ca);
      q6_codes<3>(r, t, cb);
    }
    typedef int v16i __attribute__((ext_vector_type(16)));
    const v16i zero = {};
    const v16i Ca = __builtin_amdgcn_mfma_i32_32x32x16_i8((long)x.a[e], (long)(((uint64_t)ca[1] << 32) | ca[0]), zero, 0, 0, 0);
    const v16i Cb = __builtin_amdgcn_mfma_i32_32x32x16_i8((long)x.a[e + 2], (long)(((uint64_t)cb[1] << 32) | cb[0]), zero, 0, 0, 0);
    const float sa = (float)(int)__builtin_amdgcn_sbfe((int)s4[2 * h], 8u * (uint32_t)(t + 2 * e), 8u);
    const float sb = (float)(int)__builtin_amdgcn_sbfe((int)s4[2 * h + 1], 8u * (uint32_t)(t + 2 * e), 8u);
#pragma unroll
    for (int j = 0; j < NJ; ++j)
#pragma unroll
      for (int b = 0; b < 2; ++b) {
        const int ta = (int)(((uint32_t)Ca[4 * j + 2 * b] << 7) + (uint32_t)Ca[4 * j + 2 * b + 1]);
        const int tb = (int)(((uint32_t)Cb[4 * j + 2 * b] << 7) + (uint32_t)Cb[4 * j + 2 * b + 1]);
        const int k = 2 * j + b;
        const float sx = x.sx[e][k];
        float pe = L6::fold(d, sa, sb, ta, tb) * (sx * keep);
        asm volatile("" : "+v"(pe));  // rounded before the pair add, as in the VALU kernel
        if (e == 0)
          p0[k] = pe;
        else
          P[k] = p0[k] + pe;
      }
  }
}

// Work decomposition (k_gemv_q6s, 16 waves a workgroup):
//  * Workgroup b owns 64-slot block blk = b % nb of its rows and the 32-row tiles b / nb,
//    b / nb + P, ... (P workgroups a block, about one workgroup a CU in all).  Wave w owns step w of
//    the block (the block's slot pairs 2w and 2w + 1), so its activation operands -- the
//    convert_task<2> records and steps of those two pairs for every vector -- are the same for
//    every tile: the wave converts them once, through LDS, into registers.
//  * Tiles stream through a two-stage LDS ring: a tile's block (32 rows x 1680 bytes) is copied by
//    buffer_load_dword ... lds (rows 421 dwords apart: on distinct banks) while the previous tile is
//    folded.  Each wave folds its step for the tile's 32 rows (four MFMAs a pair, the B codes built
//    from the raw bytes as dword-aligned windows realigned, as the VALU kernel reads them), and the
//    workgroup sums the 16 step sums of each output as a balanced tree.
//  * A row of one block is written as it is.  Otherwise the block sums go to the workspace and a
//    second launch (k_q6s_sum) adds each output's nb block sums in block order from 0.0f.
#define QVX_LDS __attribute__((address_space(3)))
constexpr uint32_t kQ6sRsrcWord3 = 0x00020000u;              // raw buffer, 32-bit data (gfx9)
constexpr int kQ6sRowBytes = 8 * 210;                        // a row's 64-slot block
constexpr int kQ6sRowWords = kQ6sRowBytes / 4 + 1;           // LDS dwords a staged row: odd, so 32 rows
                                                             // fall on distinct banks
constexpr int kQ6sStage = 32 * kQ6sRowWords * 4;             // LDS bytes of a ring stage
constexpr int kQ6sRowCopies = (kQ6sRowBytes / 4 + 63) / 64;  // 64-dword copies a row: 7, the last one
constexpr int kQ6sLastLanes = kQ6sRowBytes / 4 - 64 * (kQ6sRowCopies - 1);  // ... 36 lanes wide
constexpr int kQ6sWaveCopies = 2 * kQ6sRowCopies;            // copies a wave a tile (2 rows): 14

// Copy global -> LDS, 4 bytes a lane (buffer_load_dword ... lds: lane l's dword, from byte voff +
// soff of the buffer, lands at LDS byte dst + 4 l).  Written as inline asm so that the compiler,
// which does not see it as an LDS write, inserts no wait for it before LDS reads: the kernel waits
// for its copies itself (q6s_wait_vm), which lets one stage be read while the other is being copied
// into.  The s_nop is the wait state the hardware needs between the M0 write and the copy.
__device__ inline void q6s_copy4(__amdgpu_buffer_rsrc_t r, uint32_t dst, uint32_t voff, uint32_t soff) {
  asm volatile("s_nop 0\n\tbuffer_load_dword %0, %1, %2 offen lds" ::"v"(voff), "s"(r), "s"(soff), "{m0}"(dst)
               : "memory");
}
// s_waitcnt vmcnt(N), other counters untouched (gfx9 encoding); a compiler barrier for memory.
template <int N>
__device__ inline void q6s_wait_vm() {
  static_assert(N >= 0 && N < 63, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
// A 16-byte global load whose wait the kernel places itself (q6s_wait_x): the compiler, which does
// not see the load, does not wait for the ring copies issued after it before the value's first use.
typedef float q6s_f4 __attribute__((ext_vector_type(4)));
__device__ inline q6s_f4 q6s_ldx(const float* p) {
  q6s_f4 r;
  asm volatile("global_load_dwordx4 %0, %1, off" : "=v"(r) : "v"(p));
  return r;
}
// Waits until at most N vector memory operations are outstanding; the loaded values are operands,
// so no use of them moves above the wait.
template <int N>
__device__ inline void q6s_wait_x(q6s_f4* a, q6s_f4* b, int n) {
  if (n == 1)
    asm volatile("s_waitcnt vmcnt(%2)" : "+v"(a[0]), "+v"(b[0]) : "n"(N) : "memory");
  else if (n == 2)
    asm volatile("s_waitcnt vmcnt(%4)" : "+v"(a[0]), "+v"(a[1]), "+v"(b[0]), "+v"(b[1]) : "n"(N) : "memory");
  else
    asm volatile("s_waitcnt vmcnt(%8)"
                 : "+v"(a[0]), "+v"(a[1]), "+v"(a[2]), "+v"(a[3]), "+v"(b[0]), "+v"(b[1]), "+v"(b[2]), "+v"(b[3])
                 : "n"(N)
                 : "memory");
}
// Workgroup barrier for LDS only: this wave's LDS accesses complete, then s_barrier.  (__syncthreads
// would also wait for the ring's copies in flight.)
__device__ inline void q6s_lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

struct Q6sGeo {
  int nb;     // 64-slot blocks a row (cols / 2048)
  int ntile;  // 32-row tiles
  int P;      // workgroups a block
  uint32_t row_bytes;
};

// cnt (8 vectors or fewer, 2..8 blocks a row): per-tile counters that are zero on entry and are left
// zero; the block sums are then added in the kernel by the workgroup that counts a tile's last
// block in, instead of by k_q6s_sum.
template <int NV>
__global__ __launch_bounds__(1024) void k_gemv_q6s(const uint8_t* __restrict__ W, const float* __restrict__ X,
                                                   float* __restrict__ Y, int rows, int cols, int nv, Q6sGeo geo,
                                                   float* __restrict__ part, uint32_t* __restrict__ cnt) {
  static_assert(NV == 4 || NV == 8 || NV == 16, "4, 8 or 16 vectors a launch");
  using L6 = Lane<T_Q6_K>;
  constexpr int NJ = NV / 4, NO = NV * 32;
  constexpr int RW = NV * 40 + 2 * NV;  // words of one pair's converted operands: records, then steps
  static_assert(16 * 2 * RW * 4 <= kQ6sStage + 16 * NO * 4, "conversion scratch fits in stage 1 + sums");
  __shared__ __attribute__((aligned(16))) uint8_t lds[2 * kQ6sStage + (NV <= 8 ? 2 : 1) * 16 * NO * 4];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int ln = lane & 31, g = lane >> 5;
  const int blk = (int)blockIdx.x % geo.nb, pi = (int)blockIdx.x / geo.nb;
  const int ntl = pi < geo.ntile ? (geo.ntile - pi + geo.P - 1) / geo.P : 0;  // tiles of this workgroup
  const uint32_t lds_base = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(QVX_LDS uint8_t*)lds);

  // Copy of the workgroup's j-th tile into stage s: wave w copies rows 2w and 2w + 1, each row's
  // block as 7 copies of 64 dwords (the last one 36 lanes wide) into kQ6sRowWords dwords of LDS (the
  // last dword is padding, never written).  Rows past the weight repeat its last row.
  auto issue = [&](int j, int s) __attribute__((always_inline)) {
    const int r0 = (pi + j * geo.P) * 32, nr = min(32, rows - r0);
    const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(W + (size_t)r0 * geo.row_bytes), (short)0, (int)((uint32_t)nr * geo.row_bytes), (int)kQ6sRsrcWord3);
#pragma unroll
    for (int rr = 0; rr < 2; ++rr) {
      const int r = min(2 * wave + rr, nr - 1);
      const uint32_t so = (uint32_t)r * geo.row_bytes + (uint32_t)blk * kQ6sRowBytes;
      const uint32_t dst = lds_base + (uint32_t)(s * kQ6sStage + (2 * wave + rr) * kQ6sRowWords * 4);
#pragma unroll
      for (int i = 0; i < kQ6sRowCopies; ++i)
        if (i + 1 < kQ6sRowCopies || lane < kQ6sLastLanes) q6s_copy4(rsrc, dst + 256u * i, 4u * lane, so + 256u * i);
    }
  };
  if (ntl == 0) return;  // the whole workgroup

  // The wave's operands: pairs blk*32 + 2 wave + t (t = 0, 1) of every vector, converted into its
  // slice of stage 1 (not yet copied into) and read back into registers.  The activations are
  // requested before tile 0's copies and waited for with those still in flight.
  Q6Act<NV> xa[2];
  {
    constexpr int NT = 16 * NV / 64;  // conversion tasks a lane: 8 NV a pair
    uint32_t* cw = reinterpret_cast<uint32_t*>(lds + kQ6sStage) + wave * 2 * RW;
    static_assert(NT == 1 || NT == 2 || NT == 4, "one, two or four tasks a lane");
    q6s_f4 y0[NT], y1[NT];
#pragma unroll
    for (int k = 0; k < NT; ++k) {
      const int T = lane + 64 * k, t = T / (8 * NV), tt = T - t * 8 * NV;
      const int v = tt >> 3, e = (tt >> 2) & 1, part4 = tt & 3;
      const int slot = 2 * (blk * 32 + 2 * wave + t) + e;
      const float* src = X + (size_t)min(v, nv - 1) * cols + L6::xoff(slot, part4 >> 1) + 8 * (part4 & 1);
      y0[k] = q6s_ldx(src);
      y1[k] = q6s_ldx(src + 4);
    }
    issue(0, 0);
    q6s_wait_x<kQ6sWaveCopies>(y0, y1, NT);
    float4 x0[NT], x1[NT];
#pragma unroll
    for (int k = 0; k < NT; ++k) {
      const int T = lane + 64 * k, tt = T % (8 * NV);
      const bool pad = (tt >> 3) >= nv;  // padding vectors: zero records
      x0[k] = pad ? make_float4(0.0f, 0.0f, 0.0f, 0.0f) : make_float4(y0[k].x, y0[k].y, y0[k].z, y0[k].w);
      x1[k] = pad ? make_float4(0.0f, 0.0f, 0.0f, 0.0f) : make_float4(y1[k].x, y1[k].y, y1[k].z, y1[k].w);
    }
#pragma unroll
    for (int k = 0; k < NT; ++k) {
      const int T = lane + 64 * k, t = T / (8 * NV), tt = T - t * 8 * NV;
      const int v = tt >> 3, e = (tt >> 2) & 1;
      uint32_t* rw = cw + t * RW;
      float* so = reinterpret_cast<float*>(rw + NV * 40) + e * NV + ((v >> 1) & 1) * (NV / 2) + 2 * (v >> 2) + (v & 1);
      convert_task<2>(x0[k], x1[k], tt, true, rw, so);
    }
#pragma unroll
    for (int t = 0; t < 2; ++t)
      q6_act_load<NV>(cw + t * RW, 40, reinterpret_cast<const float*>(cw + t * RW + NV * 40), lane, xa[t]);
  }
  // every wave's operands are in registers: stage 1 is free (the 16-vector loop copies tile 1 into
  // it now; the 8-vector loop at the top of tile 0)
  q6s_lds_barrier();
  if (NV != 8 && ntl > 1) issue(1, 1);

  const int sbk = wave >> 1, h = wave & 1;  // the wave's super-block of the block, half
  const uint32_t pb = (uint32_t)sbk * 210u;
  auto read_tile = [&](int s, Q6Half& hw) __attribute__((always_inline)) {
    const uint8_t* base = lds + s * kQ6sStage + ln * (4 * kQ6sRowWords) + pb;
    q6_load_codes(base, pb & 3u, g, h, hw);
    q6_load_scales(base, pb & 3u, hw);
  };
  auto fold_tile = [&](const Q6Half& hw, float* rb) __attribute__((always_inline)) {
    float P0[NV / 2], P1[NV / 2];
    q6_pair_fold<NV>(hw, h, 0, xa[0], lane, P0);
    q6_pair_fold<NV>(hw, h, 1, xa[1], lane, P1);
#pragma unroll
    for (int jj = 0; jj < NJ; ++jj)
#pragma unroll
      for (int b = 0; b < 2; ++b) rb[wave * NO + (4 * jj + 2 * g + b) * 32 + ln] = P0[2 * jj + b] + P1[2 * jj + b];
  };
  // The block sum of each output o = (vector, row) of the workgroup's jt-th tile: the balanced tree
  // over the 16 step sums, four threads an output -- thread k adds steps 4k..4k+3 (a unit), then
  // the four units (U0 + U1) + (U2 + U3) across the quad (commutative adds: every lane of the quad
  // holds the same bits).
  auto combine = [&](int jt, const float* rb) __attribute__((always_inline)) {
    const int tile = pi + jt * geo.P;
#pragma unroll
    for (int o4 = tid; o4 < 4 * NO; o4 += 1024) {
      const int o = o4 >> 2, k = o4 & 3;
      float u = (rb[(4 * k) * NO + o] + rb[(4 * k + 1) * NO + o]) + (rb[(4 * k + 2) * NO + o] + rb[(4 * k + 3) * NO + o]);
      u = u + dpp<kXor1>(u);
      u = u + dpp<kXor2>(u);
      if (k == 0) {
        const int v = o >> 5, r = tile * 32 + (o & 31);
        if (geo.nb == 1) {
          if (v < nv && r < rows) Y[(size_t)v * rows + r] = u;
        } else if (cnt) {  // device-coherent: read back by the tile's last workgroup in this launch
          __hip_atomic_store(part + ((size_t)tile * geo.nb + blk) * NO + o, u, __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
        } else {  // read back by the sum launch
          part[((size_t)tile * geo.nb + blk) * NO + o] = u;
        }
      }
    }
  };

  // Tile j.  With 4 or 8 vectors: one barrier a tile, after which tile j + 1 is copied into the other
  // stage (whose tile j - 1 every wave has read), tile j is read and folded into one of two
  // step-sum buffers, and the block sums of tile j - 1 are formed from the other.  With 16 (room for
  // one buffer): tile j + 2 is copied once every wave has read tile j, and tile j's block sums are
  // formed after a second barrier.
  float* res = reinterpret_cast<float*>(lds + 2 * kQ6sStage);
  // In-kernel sums (cnt): tile jt's block sums are stored during tile jt + 1.  During tile jt + 2
  // (every wave has waited for its stores and passed the barrier) thread 0 counts the workgroup in
  // with a wrapping increment, which leaves the counter zero again after the tile's last workgroup;
  // at the top of tile jt + 3 (the ticket has arrived with that tile's wait) it posts whether the
  // workgroup was the last, and that workgroup then loads the nb block sums of each output, adds them
  // in block order from 0.0f after the fold and stores the outputs.  The loads follow the ticket
  // through the LDS flag and a barrier (the protocol of split_k_last).
  __shared__ int lastf[2];
  const bool fin = NV <= 8 && cnt != nullptr;
  auto tile_of = [&](int jt) { return pi + jt * geo.P; };
  auto ticket = [&](int jt) __attribute__((always_inline)) {
    return __builtin_amdgcn_atomic_inc32(cnt + tile_of(jt), (uint32_t)(geo.nb - 1), __ATOMIC_RELAXED, "agent");
  };
  auto final_loads = [&](int jt, float (&fv)[8]) __attribute__((always_inline)) {
    const float* tp = part + (size_t)tile_of(jt) * geo.nb * NO + tid;
#pragma unroll
    for (int k = 0; k < 8; ++k)
      fv[k] = __hip_atomic_load(tp + (size_t)min(k, geo.nb - 1) * NO, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  };
  auto final_store = [&](int jt, const float (&fv)[8]) __attribute__((always_inline)) {
    float sum = 0.0f;
#pragma unroll
    for (int k = 0; k < 8; ++k)
      if (k < geo.nb) sum += fv[k];
    const int v = tid >> 5, r = tile_of(jt) * 32 + (tid & 31);
    if (v < nv && r < rows) Y[(size_t)v * rows + r] = sum;
  };
  uint32_t tkt = 0;
  for (int j = 0; j < ntl; ++j) {
    const int s = j & 1;
    Q6Half hw;
    if constexpr (NV <= 8) {
      q6s_wait_vm<0>();  // tile j's copies (and the stores, loads and ticket issued since)
      if (fin && j >= 3 && tid == 0) lastf[j & 1] = tkt == (uint32_t)(geo.nb - 1) ? 1 : 0;  // tile j - 3
      q6s_lds_barrier();
      if (j + 1 < ntl) issue(j + 1, s ^ 1);
      read_tile(s, hw);
      if (fin && j >= 2 && tid == 0) tkt = ticket(j - 2);
      const bool fl = fin && j >= 3 && lastf[j & 1] != 0;  // this workgroup sums tile j - 3
      float fv[8];
      if (fl && tid < NO) final_loads(j - 3, fv);
      if (j > 0) combine(j - 1, res + ((j - 1) & 1) * 16 * NO);
      fold_tile(hw, res + (j & 1) * 16 * NO);
      if (fl && tid < NO) final_store(j - 3, fv);
    } else {
      // this wave's copies of tile j are done when at most tile j + 1's are still in flight (loads
      // complete in order; the block-sum stores in between are not counted: they may complete in
      // any order)
      if (j + 1 < ntl) q6s_wait_vm<kQ6sWaveCopies>();
      else q6s_wait_vm<0>();
      q6s_lds_barrier();
      read_tile(s, hw);
      fold_tile(hw, res);
      q6s_lds_barrier();  // stage s has been read, the step sums are complete
      if (j + 2 < ntl) issue(j + 2, s);
      combine(j, res);
    }
  }
  if constexpr (NV <= 8) {
    const int J = ntl;
    q6s_lds_barrier();  // the last fold is done
    combine(J - 1, res + ((J - 1) & 1) * 16 * NO);
    if (fin) {
      // tiles J - 3 (its ticket is in flight), J - 2 and J - 1 (their stores complete with this wait)
      q6s_wait_vm<0>();
      if (tid == 0) {
        lastf[0] = J >= 3 && tkt == (uint32_t)(geo.nb - 1) ? 1 : 0;
        lastf[1] = J >= 2 && ticket(J - 2) == (uint32_t)(geo.nb - 1) ? 1 : 0;
      }
      __shared__ int lastf2;
      if (tid == 0) lastf2 = ticket(J - 1) == (uint32_t)(geo.nb - 1) ? 1 : 0;
      q6s_lds_barrier();
      const int fl3[3] = {lastf[0], lastf[1], lastf2};
#pragma unroll
      for (int t = 0; t < 3; ++t) {
        if (fl3[t] == 0 || tid >= NO) continue;
        float fv[8];
        final_loads(J - 3 + t, fv);
        final_store(J - 3 + t, fv);
      }
    }
  }
}

// out[v, r] = the nb block sums of (v, r) added in block order from 0.0f (NO = 32 x the launch's
// padded vector count; part as k_gemv_q6s writes it).
__global__ __launch_bounds__(256) void k_q6s_sum(const float* __restrict__ part, float* __restrict__ Y, int rows,
                                                 int nv, int nb, int NO, int ntile) {
  const int idx = (int)blockIdx.x * 256 + (int)threadIdx.x;
  if (idx >= ntile * NO) return;
  const int tile = idx / NO, o = idx - tile * NO, v = o >> 5, r = tile * 32 + (o & 31);
  if (v >= nv || r >= rows) return;
  const float* p = part + (size_t)tile * nb * NO + o;
  float sum = 0.0f;
  for (int k0 = 0; k0 < nb; k0 += 8) {  // eight block sums in flight at a time, added in order
    float b8[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) b8[k] = p[(size_t)min(k0 + k, nb - 1) * NO];
#pragma unroll
    for (int k = 0; k < 8; ++k)
      if (k0 + k < nb) sum += b8[k];
  }
  Y[(size_t)v * rows + r] = sum;
}

int device_cus();

inline Q6sGeo q6s_geometry(int rows, int cols, size_t row_bytes) {
  Q6sGeo geo;
  geo.nb = cols / 2048;
  geo.ntile = (rows + 31) / 32;
  geo.P = std::max(1, std::min(geo.ntile, device_cus() / geo.nb));
  geo.row_bytes = (uint32_t)row_bytes;
  return geo;
}

// 1 if the batched form takes the shape (K a multiple of 2048, row pitch below 4 GiB), and its
// workspace bytes for nvec vectors through *ws_bytes (the block sums; none for rows of one block).
inline int q6s_nvp(int nvec) { return nvec <= 4 ? 4 : nvec <= 8 ? 8 : 16; }
bool gemv_q6s_route(int nvec, int rows, int cols, size_t row_bytes, size_t* ws_bytes) {
  if (cols <= 0 || cols % 2048 != 0 || rows <= 0 || nvec <= 0 || row_bytes > 0xFFFFFFFFull / 64) return false;
  if (ws_bytes) {
    const int nb = cols / 2048;
    *ws_bytes = nb > 1 ? (size_t)((rows + 31) / 32) * nb * q6s_nvp(nvec) * 32 * 4 : 0;
  }
  return true;
}

// Tile counters a call can use to add its block sums in the kernel: one a 32-row tile; 0 where the
// call has no use for them.  Only launches of 8 vectors or fewer with 2..8 blocks a row whose
// workgroups take at most 2 tiles each use them: measured, they save the sum launch there (1024 x
// 4096 at M = 8: 8.4 -> 7.4 us, 4096 x 4096: 9.7 -> 8.5) but cost more than it on deeper loops (4096
// x 14336 at M = 8, 4 tiles a workgroup: 19.6 -> 20.1; the LM head at M = 4: 88 -> 97), where the
// workgroups that come last on several tiles stretch the tail.
int gemv_q6s_counters(int nvec, int rows, int cols) {
  const int nb = cols / 2048, ntile = (rows + 31) / 32;
  if (q6s_nvp(nvec) > 8 || nb < 2 || nb > 8) return 0;
  const int P = std::max(1, std::min(ntile, device_cus() / nb));
  return (ntile + P - 1) / P <= 2 ? ntile : 0;
}

// qmatmul_n over Q6_K on the batched form, 16 vectors a launch (8 or 4 when the whole call has at most
// 8 or 4), each launch followed by the in-order sum of its block sums when rows have several blocks:
// in the kernel when the call brings zeroed tile counters (cnt: gemv_q6s_counters of them, zero on
// entry and left zero -- a plan's), else in a launch of its own.
bool launch_gemv_q6s(const void* w, const float* X, float* Y, int nvec, int rows, int cols, size_t row_bytes,
                     void* ws, hipStream_t s, uint32_t* cnt) {
  if (!gemv_q6s_route(nvec, rows, cols, row_bytes, nullptr)) return false;
  const Q6sGeo geo = q6s_geometry(rows, cols, row_bytes);
  if (geo.nb > 1 && !ws) return false;
  const int nvp = q6s_nvp(nvec), NO = nvp * 32;
  const auto* wb = static_cast<const uint8_t*>(w);
  auto* part = static_cast<float*>(ws);
  if (gemv_q6s_counters(nvec, rows, cols) == 0) cnt = nullptr;
  const unsigned grid = (unsigned)(geo.nb * geo.P);
  for (int v0 = 0; v0 < nvec; v0 += nvp) {
    const int nv = std::min(nvp, nvec - v0);
    const float* Xv = X + (size_t)v0 * cols;
    float* Yv = Y + (size_t)v0 * rows;
    if (nvp == 4) k_gemv_q6s<4><<<grid, 1024, 0, s>>>(wb, Xv, Yv, rows, cols, nv, geo, part, cnt);
    else if (nvp == 8) k_gemv_q6s<8><<<grid, 1024, 0, s>>>(wb, Xv, Yv, rows, cols, nv, geo, part, cnt);
    else k_gemv_q6s<16><<<grid, 1024, 0, s>>>(wb, Xv, Yv, rows, cols, nv, geo, part, nullptr);
    if (geo.nb > 1 && !cnt)
      k_q6s_sum<<<(unsigned)((geo.ntile * NO + 255) / 256), 256, 0, s>>>(part, Yv, rows, nv, geo.nb, NO, geo.ntile);
  }
  return true;
}

// ---- launch ---------------------------------------------------------------------------------

template <uint32_t T, int NV, int RMAX, int TPT, bool CH, bool NORM>
static bool launch_t(const void* w, const float* X, float* Y, int rows, int cols, const Geo& geo, int nwg,
                     const GemvEpi& epi, hipStream_t s) {
  constexpr int PF = prefetch_rows<T, NV>() < RMAX ? prefetch_rows<T, NV>() : RMAX;
  auto kern = &k_gemv<T, NV, RMAX, TPT, PF, CH, NORM>;
  const size_t lds = gemv_lds_bytes<T>(NV, geo.S);
  static LdsLimit lim;
  if (!lds_ready(reinterpret_cast<const void*>(kern), lim, lds)) return false;
  kern<<<(unsigned)nwg, dim3((unsigned)geo.Sp, (unsigned)geo.G), lds, s>>>(static_cast<const uint8_t*>(w), X, Y,
                                                                           rows, cols, geo, epi.norm_w, epi.eps);
  return true;
}

// Rows per group RMAX (1..RM), rounded up to an instantiated value.
template <uint32_t T, int NV, int TPT, int RM, bool NORM>
static bool launch_r(int rmax, const void* w, const float* X, float* Y, int rows, int cols, const Geo& geo, int nwg,
                     const GemvEpi& epi, hipStream_t s) {
  if constexpr (RM > 1) {
    if (rmax < RM) return launch_r<T, NV, TPT, RM - 1, NORM>(rmax, w, X, Y, rows, cols, geo, nwg, epi, s);
  }
  return launch_t<T, NV, RM, TPT, false, NORM>(w, X, Y, rows, cols, geo, nwg, epi, s);
}

template <uint32_t T, int NV, int TPT, bool NORM>
static bool launch_tpt(const void* w, const float* X, float* Y, int rows, int cols, Geo geo, const GemvEpi& epi,
                       hipStream_t s) {
  constexpr int rm = max_rows<NV, TPT>();
  static_assert(rm % prefetch_rows<T, NV>() == 0, "chunks of rm rows keep the prefetch ring aligned");
  int per_group = 0;
  const int nwg = valu_grid(rows, geo, per_group);
  if (per_group <= rm) return launch_r<T, NV, TPT, rm, NORM>(per_group, w, X, Y, rows, cols, geo, nwg, epi, s);
  return launch_t<T, NV, rm, TPT, true, NORM>(w, X, Y, rows, cols, geo, nwg, epi, s);
}

template <uint32_t T, int NV, bool NORM>
static bool launch_nv2(const void* w, const float* X, float* Y, int rows, int cols, const Geo& geo,
                       const GemvEpi& epi, hipStream_t s) {
  const int threads = geo.G * geo.Sp;
  const int tpt = (NV * geo.S * 2 * Lane<T>::kR + threads - 1) / threads;
  if (tpt > 8) return false;  // the kernel converts at most 8 tasks a thread
  if (tpt <= 1) return launch_tpt<T, NV, 1, NORM>(w, X, Y, rows, cols, geo, epi, s);
  if (tpt <= 2) return launch_tpt<T, NV, 2, NORM>(w, X, Y, rows, cols, geo, epi, s);
  if (tpt <= 4) return launch_tpt<T, NV, 4, NORM>(w, X, Y, rows, cols, geo, epi, s);
  return launch_tpt<T, NV, 8, NORM>(w, X, Y, rows, cols, geo, epi, s);
}
template <uint32_t T, int NV>
static bool launch_nv(const void* w, const float* X, float* Y, int rows, int cols, const Geo& geo,
                      const GemvEpi& epi, hipStream_t s) {
  Geo g = geo;
  g.G = gemv_threads<T, NV>() / geo.Sp;  // the caller checked Sp <= the workgroup's threads
  return epi.norm_w ? launch_nv2<T, NV, true>(w, X, Y, rows, cols, g, epi, s)
                    : launch_nv2<T, NV, false>(w, X, Y, rows, cols, g, epi, s);
}

template <uint32_t T>
static bool launch_type(const void* w, const float* X, float* Y, int nvec, int rows, int cols, const Geo& geo,
                        const GemvEpi& epi, hipStream_t s) {
  // Four vectors a launch when their activations fit in LDS, so the weights are streamed once per
  // four vectors instead of once per two: Q6_K at 1024 threads, the other formats at 512 (groups
  // of up to 512 lanes).
  constexpr int thr4 = gemv_threads<T, 4>();
  const bool nv4 = gemv_lds_bytes<T>(4, geo.S) <= 150 * 1024 && geo.Sp <= thr4 &&
                   4 * geo.S * 2 * Lane<T>::kR <= 8 * thr4;  // at most 8 conversion tasks a thread
  for (int v0 = 0; v0 < nvec;) {
    const float* Xv = X + (size_t)v0 * cols;
    float* Yv = Y + (size_t)v0 * rows;
    const int left = nvec - v0;
    if (nv4 && left >= 4) {
      if (!launch_nv<T, 4>(w, Xv, Yv, rows, cols, geo, epi, s)) return false;
      v0 += 4;
      continue;
    }
    if (left >= 2) {
      if (!launch_nv<T, 2>(w, Xv, Yv, rows, cols, geo, epi, s)) return false;
      v0 += 2;
    } else {
      if (!launch_nv<T, 1>(w, Xv, Yv, rows, cols, geo, epi, s)) return false;
      v0 += 1;
    }
  }
  return true;
}

template <uint32_t T>
static bool launch_fast_t(const void* w, const float* X, float* Y, int nvec, int rows, int cols, size_t row_bytes,
                          const GemvEpi& epi, hipStream_t s) {
  Geo geo{};
  if (!geometry<T>(cols, row_bytes, geo)) return false;
  if (epi.swiglu) return false;
  if (epi.norm_w && (cols % kNormChunk != 0 || cols / kNormChunk > kNormMaxChunks)) return false;
  return launch_type<T>(w, X, Y, nvec, rows, cols, geo, epi, s);
}

// 1 if launch_gemv_fast takes this shape together with the fused prologue `epi` (RMSNorm only:
// this kernel's outputs are plain rows), so a fused call can be routed here before anything runs.
bool gemv_fast_fusable(uint32_t t, int cols, size_t row_bytes, const GemvEpi& epi) {
  if (epi.swiglu) return false;
  if (epi.norm_w && (cols % kNormChunk != 0 || cols / kNormChunk > kNormMaxChunks)) return false;
  Geo geo{};
  switch (t) {
    case T_Q4_K: return geometry<T_Q4_K>(cols, row_bytes, geo);
    case T_Q6_K: return geometry<T_Q6_K>(cols, row_bytes, geo);
    case T_Q5_K: return geometry<T_Q5_K>(cols, row_bytes, geo);
    case T_Q4_0: return geometry<T_Q4_0>(cols, row_bytes, geo);
    case T_Q5_0: return geometry<T_Q5_0>(cols, row_bytes, geo);
    case T_Q8_0: return geometry<T_Q8_0>(cols, row_bytes, geo);
    default: return false;
  }
}

// Fast-path GEMV for nvec >= 1 on 16-byte-aligned rows of Q8_0 / Q4_0 / Q5_0 / Q4_K / Q5_K / Q6_K.  Returns
// false, having launched nothing, when the shape needs the generic kernel.
bool launch_gemv_fast(uint32_t t, const void* w, const float* X, float* Y, int nvec, int rows, int cols,
                      size_t row_bytes, const GemvEpi& epi, hipStream_t s) {
  switch (t) {
    case T_Q4_K: return launch_fast_t<T_Q4_K>(w, X, Y, nvec, rows, cols, row_bytes, epi, s);
    case T_Q6_K: return launch_fast_t<T_Q6_K>(w, X, Y, nvec, rows, cols, row_bytes, epi, s);
    case T_Q5_K: return launch_fast_t<T_Q5_K>(w, X, Y, nvec, rows, cols, row_bytes, epi, s);
    case T_Q4_0: return launch_fast_t<T_Q4_0>(w, X, Y, nvec, rows, cols, row_bytes, epi, s);
    case T_Q5_0: return launch_fast_t<T_Q5_0>(w, X, Y, nvec, rows, cols, row_bytes, epi, s);
    case T_Q8_0: return launch_fast_t<T_Q8_0>(w, X, Y, nvec, rows, cols, row_bytes, epi, s);
    default: return false;
  }
}

}  // namespace qvx
