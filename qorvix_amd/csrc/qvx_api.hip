// qvx_api.hip -- the extern "C" boundary of libqvx.so (declared in include/qvx.h).
//
// Argument checks mirror the reference's operator (runtime/src/qmatmul.cpp:24-126) one for one
// and run before any device work; then the call dispatches on the ggml type to the gfx950
// kernels.  The engine never falls back to the CPU: a missing device or a failed launch is an
// error code.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstring>
#include <mutex>
#include <new>
#include <vector>

#include "../../include/qvx.h"
#include "qvx_common.hpp"
#include "qvx_norm.hpp"

#include <algorithm>

namespace qvx {
bool launch_dequant(uint32_t t, const void* src, float* dst, size_t n, hipStream_t s);
bool launch_gemv_generic(uint32_t t, const void* w, const float* X, float* Y, int rows, int cols, int nvec,
                         size_t row_bytes, hipStream_t s);
bool launch_gemv_fast(uint32_t t, const void* w, const float* X, float* Y, int nvec, int rows, int cols,
                      size_t row_bytes, const GemvEpi& epi, hipStream_t s);
bool gemv_fast_fusable(uint32_t t, int cols, size_t row_bytes, const GemvEpi& epi);
bool mx_epi_supported(const GemvEpi& epi, int rows, int cols);
void launch_rmsnorm(float* out, const float* x, const float* w, float eps, int nvec, int n, hipStream_t s);
void launch_swiglu(float* out, const float* g, const float* u, size_t n, hipStream_t s);
void launch_swiglu_interleaved(float* out, const float* y, int nvec, int ffn, hipStream_t s);
void* gemm_temp_alloc(size_t bytes, hipStream_t s);
void gemm_temp_free(void* p, hipStream_t s);
bool launch_gemv_float(uint32_t t, const void* w, const float* X, float* Y, int nvec, int rows, int cols,
                       size_t row_bytes, hipStream_t s);
int gemv_mx_max_nv(int cols);
int gemv_mxj_supported(int cols);
bool launch_gemv_mxj_q4k(const void* w, const float* X, float* Y, int nvec, int rows, int cols, size_t row_bytes,
                         hipStream_t s);
bool launch_gemv_mx_q4k(const void* w, const float* X, float* Y, int nvec, int rows, int cols, size_t row_bytes,
                        const GemvEpi& epi, hipStream_t s);
int gemv_mxb_supported(int cols);
bool launch_gemv_mxb_q4k(const void* w, const float* X, float* Y, int nvec, int rows, int cols, size_t row_bytes,
                         const GemvEpi& epi, hipStream_t s);
bool launch_fill_synthetic(void* w, uint32_t t, size_t nblk, uint64_t seed, float mul, hipStream_t s);
void launch_fill_normal_f32(float* x, size_t n, uint64_t seed, float mul, hipStream_t s);
void launch_fill_normal_f16(uint16_t* x, size_t n, uint64_t seed, float mul, hipStream_t s);
void launch_read16(const void* src, size_t n16, uint32_t* flag, hipStream_t s);
bool qgemm_deq_supported(uint32_t t, const void* w, const uint16_t* X, int K, int N, size_t row_bytes);
int q4k_plan_desc(int M, int N, int K, int cus, int* desc, int cap);
bool gemv_q6s_route(int nvec, int rows, int cols, size_t row_bytes, size_t* ws_bytes);
bool gemv_q4s_route(int nvec, int rows, int cols, size_t row_bytes, size_t* ws_bytes);
bool launch_gemv_q4s(const void* w, const float* X, float* Y, const float* bias, int nvec, int rows, int cols,
                     size_t row_bytes, void* ws, hipStream_t s);
bool launch_gemv_q6s(const void* w, const float* X, float* Y, int nvec, int rows, int cols, size_t row_bytes,
                     void* ws, hipStream_t s, uint32_t* cnt);
int gemv_q6s_counters(int nvec, int rows, int cols);
int launch_qgemm(float* out, const void* w, uint32_t t, const uint16_t* X, int M, int rows, int cols,
                 int variant, hipStream_t s, void* ws, size_t ws_cap);
int launch_gemm16_entry(float* out, const uint16_t* X, const uint16_t* B, int M, int N, int K, bool bf16,
                        hipStream_t s);
bool launch_dequant16(uint32_t t, const void* src, uint16_t* dst, size_t n, bool bf16, hipStream_t s);
int launch_quantize_act_q8(const uint16_t* X, int M, int K, int8_t* q, float* scale, int32_t* qsum,
                           hipStream_t s);
void launch_zero(float* p, size_t n, hipStream_t s);
bool launch_gemv_group(const GemvMember* m, int n, const float* X, int cols, const GemvEpi& epi, hipStream_t s);
size_t gemv_many_ws_bytes(int nvec, int rows, int cols, size_t row_bytes);
int gemv_many_supported(int cols, size_t row_bytes);
bool launch_gemv_q4k_many(const void* w, const float* X, float* Y, const float* bias, int nvec, int rows, int cols,
                          size_t row_bytes, void* ws, hipStream_t s);
void launch_add_bias(float* out, const float* bias, int nvec, int rows, hipStream_t s);
}  // namespace qvx

using namespace qvx;

// Scratch of qvx_qgemm_f16_noalloc: one fixed array per device, held from the library's first use
// on that device until the process ends.  In host code `scratch` names a host-side stand-in, not the
// device array, so kernels receive its device address, resolved once per device with
// hipGetSymbolAddress (each device holds its own copy at its own address) and used everywhere
// host code hands the array's memory to the device.
constexpr size_t kScratchBytes = (size_t)QVX_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

// A recorded GEMV sequence (include/qvx.h, qvx_plan_*).
struct qvx_plan {
  struct Call {
    float* out;
    const void* w;
    uint32_t type;
    const float* X;
    int nvec, rows, cols;
    int group;  // calls sharing a group >= 0 are independent of each other (one fork); -1: in order
    GemvEpi epi;  // fused RMSNorm / SwiGLU (rows = the weight's rows: 2 ffn for SwiGLU)
    std::vector<GemvMember> members;  // non-empty: a grouped call over X (nvec 1), out / w / type / rows unused
    size_t ws_off = 0, ws_bytes = 0;  // its slice of the plan's workspace (forms that take one)
    size_t cnt_off = 0;               // its zeroed counters (cnt_n), a slice no other call shares
    int cnt_n = 0;
  };
  std::vector<Call> calls;
  void* ws = nullptr;  // device workspace of the recorded calls, allocated by qvx_plan_instantiate
  int device = 0;
  int open_group = -1;  // the fork being recorded, -1 if none
  int groups = 0;
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
};

namespace {

constexpr int kMaxBlock = 256;  // largest block the operator accepts (qmatmul.cpp:11)
// Whether a Q6_K batch takes the matrix-core form (measured crossovers against the VALU kernel, four
// vectors a launch, on MI355X, graph-replayed): from 5 vectors, and from 3 (the VALU kernel's
// three-vector calls are slow: 4096 x 4096 10.0 against 8.5 us); at 4 on weights of >= 8192 rows or
// columns (4096 x 14336: 18.5 against 27.5 us; 4096 x 4096: 8.5 against 7.5); at 2 on weights of
// >= 65536 rows (128256 x 4096: 88 against 99 us).
inline bool q6_batched(int nvec, int rows, int cols) {
  if (nvec >= 5 || nvec == 3) return true;
  if (nvec == 4) return cols >= 8192 || rows >= 8192;
  return nvec == 2 && rows >= 65536;
}

inline hipStream_t as_stream(void* s) { return static_cast<hipStream_t>(s); }

inline int hip_status() {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    std::fprintf(stderr, "qvx: HIP error %d (%s)\n", (int)e, hipGetErrorString(e));
    return QVX_E_HIP;
  }
  return QVX_OK;
}

// A kernel launcher declined a call that passed the argument checks: its launch could not be
// configured (the kernel's LDS limit could not be raised, or its LDS plan would exceed the CU's
// 160 KiB).  That is a runtime failure, not a property of the type.
inline int refused() {
  (void)hipGetLastError();
  std::fprintf(stderr, "qvx: no kernel launch could be configured for this call\n");
  return QVX_E_HIP;
}

// Shape checks shared by qmatmul / qmatmul_n / qgemm: the reference's order of tests.
inline int check_matmul(uint32_t type, int cols, const TypeInfo** ti) {
  const TypeInfo* t = type_info(type);
  if (!t || !can_dequantize(type) || !gemv_supports(type)) return QVX_E_TYPE;
  if (t->block == 0 || (int)t->block > kMaxBlock || cols % (int)t->block != 0) return QVX_E_SHAPE;
  *ti = t;
  return QVX_OK;
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Whether a Q4_K batch takes the many-vector form rather than chunks of 8 vectors.  The form costs
// a conversion launch and a K-range chain per wave whatever the batch (17-22 us in graph replays on
// MI355X), against ~10 us per 8-vector chunk of a 4096 x 4096 weight and 14-26 us of a 58.7 M-element
// one: measured, it wins from 12 vectors on weights of >= 32 Mi elements (14336 x 4096 at 12: 20.2
// against 24.3 us; 4096 x 14336: 32.8 against 41.4), and on smaller weights only from ~24 (4096 x
// 4096 at 16: 22 against 19 us).
inline bool many_batch(int nvec, int rows, int cols) {
  return nvec >= 24 || (nvec >= 12 && (int64_t)rows * cols >= ((int64_t)32 << 20));
}

// Q4_K: the vector count a chunk may have on the one-vector matrix-core kernel before the batched
// forms take over (measured faster there), and whether the whole-row batched form takes the row.

inline int q4k_small(int cols) { return std::min(gemv_mxb_supported(cols) ? 3 : 2, gemv_mx_max_nv(cols)); }

// 1 if the routing below sends every chunk of this call to a kernel that folds `epi` in.
bool fused_route(uint32_t type, int nvec, int rows, int cols, size_t row_bytes, bool fast, const GemvEpi& epi) {
  if (!fast) return false;
  if (type == T_Q4_K && gemv_mx_max_nv(cols) > 0) {
    if (!mx_epi_supported(epi, rows, cols)) return false;
    return nvec == 1 || gemv_mxb_supported(cols) || nvec <= q4k_small(cols);
  }
  return gemv_fast_fusable(type, cols, row_bytes, epi);
}

int gemv(float* out, const void* w, uint32_t type, const float* X, int nvec, int rows, int cols, hipStream_t s,
         const GemvEpi& epi = {});

// A fused call no kernel folds in: the standalone norm into a temporary, the plain product (into a
// temporary for SwiGLU), then the de-interleaving SwiGLU.  Temporaries come from the library's
// stream-ordered pool.
int gemv_unfused(float* out, const void* w, uint32_t type, const float* X, int nvec, int rows, int cols,
                 hipStream_t s, const GemvEpi& epi) {
  const float* xin = X;
  float* xn = nullptr;
  float* y = nullptr;
  if (epi.norm_w) {
    if (cols > kNormChunk * kNormMaxChunks) return QVX_E_RANGE;
    xn = static_cast<float*>(gemm_temp_alloc((size_t)nvec * (size_t)cols * sizeof(float), s));
    if (!xn) return QVX_E_HIP;
    launch_rmsnorm(xn, X, epi.norm_w, epi.eps, nvec, cols, s);
    xin = xn;
  }
  float* dst = out;
  if (epi.swiglu) {
    y = static_cast<float*>(gemm_temp_alloc((size_t)nvec * (size_t)rows * sizeof(float), s));
    if (!y) {
      gemm_temp_free(xn, s);
      return QVX_E_HIP;
    }
    dst = y;
  }
  int rc = gemv(dst, w, type, xin, nvec, rows, cols, s);
  if (rc == QVX_OK && epi.swiglu) {
    launch_swiglu_interleaved(out, y, nvec, rows / 2, s);
    rc = hip_status();
  }
  gemm_temp_free(xn, s);
  gemm_temp_free(y, s);
  return rc;
}

// out = W . x per vector, optionally with the activations normalised (epi.norm_w) and / or the
// interleaved gate|up rows gated (epi.swiglu: rows / 2 outputs a vector).  The argument checks are
// the plain operator's.
// Whether a Q4_K batch takes the split form (k_gemv_q4s) rather than the many-vector form or chunks
// of 8 on the one-vector / batched forms.  Measured on MI355X (graph-replayed): it wins on long rows
// from 5 vectors (4096 x 14336 at 8: 20.5 against 26.0 us, at 16: 28.8 against 34.0 on the
// many-vector form; at 4: 20.1 against 17.1) and on small weights from 12 (1024 x 4096 at 16: 12.7
// against 17.6), up to 23 vectors; on 4096-element rows of larger weights the other forms are faster
// (14336 x 4096 at 8: 17.7 against 14.3).  Its fixed cost (a conversion per workgroup, the partial
// sums' launch) is ~9 us.
inline bool q4s_batch(int nvec, int rows, int cols) {
  if (nvec > 23) return false;
  return (cols >= 8192 && nvec >= 5) || ((int64_t)rows * cols <= ((int64_t)4 << 20) && nvec >= 12);
}

// Q6_K batches with the RMSNorm prologue: the standalone norm (the engine's canonical sum of squares
// and x * scale * w, so the normalised activations are the bits the VALU kernel folds in) into the
// workspace, then the batched form on them -- where the extra norm launch pays: on weights of >= 8192
// rows or columns wherever the batched form takes the call, on smaller ones from 6 vectors (below
// that the VALU kernel's launches with the norm folded in are as fast).
inline size_t ws_align(size_t n) { return (n + 255) & ~size_t(255); }
inline bool q6_norm_batched(int nvec, int rows, int cols) {
  return q6_batched(nvec, rows, cols) && (nvec >= 6 || rows >= 8192 || cols >= 8192);
}

// The forms that take a workspace, and the bytes of the one a call takes (0: none).
enum WsForm { WS_NONE, WS_MANY, WS_Q4S, WS_Q6S, WS_Q6S_NORM };
inline WsForm ws_route(uint32_t type, int nvec, int rows, int cols, size_t row_bytes, bool fast, const GemvEpi& epi,
                       size_t* bytes) {
  *bytes = 0;
  if (!fast || rows <= 0 || cols <= 0) return WS_NONE;
  if (epi.flags()) {
    if (type == T_Q6_K && epi.flags() == EPI_NORM && q6_norm_batched(nvec, rows, cols) &&
        gemv_fast_fusable(type, cols, row_bytes, epi) && gemv_q6s_route(nvec, rows, cols, row_bytes, bytes)) {
      *bytes += ws_align((size_t)nvec * (size_t)cols * sizeof(float));
      return WS_Q6S_NORM;
    }
    *bytes = 0;
    return WS_NONE;
  }
  if (type == T_Q4_K) {
    if (q4s_batch(nvec, rows, cols) && gemv_q4s_route(nvec, rows, cols, row_bytes, bytes)) return WS_Q4S;
    if (many_batch(nvec, rows, cols) && gemv_many_supported(cols, row_bytes)) {
      *bytes = gemv_many_ws_bytes(nvec, rows, cols, row_bytes);
      return WS_MANY;
    }
    *bytes = 0;
    return WS_NONE;
  }
  if (type == T_Q6_K && q6_batched(nvec, rows, cols) && gemv_q6s_route(nvec, rows, cols, row_bytes, bytes) && *bytes)
    return WS_Q6S;
  *bytes = 0;
  return WS_NONE;
}
int gemv(float* out, const void* w, uint32_t type, const float* X, int nvec, int rows, int cols, hipStream_t s,
         const GemvEpi& epi) {
  const TypeInfo* ti = nullptr;
  if (nvec <= 0) return QVX_E_NVEC;
  if (int rc = check_matmul(type, cols, &ti); rc != QVX_OK) return rc;
  if (rows <= 0) return QVX_OK;
  if (!out) return QVX_E_NULL;
  const int nout = epi.swiglu ? rows / 2 : rows;
  if (cols <= 0) {  // no columns: every dot product is empty (the reference writes 0.0f; silu(0) * 0 = 0)
    launch_zero(out, (size_t)nout * (size_t)nvec, s);
    if (epi.bias) launch_add_bias(out, epi.bias, nvec, rows, s);
    return hip_status();
  }
  if (!w || !X) return QVX_E_NULL;
  const size_t row_bytes = (size_t)(cols / (int)ti->block) * ti->bytes;
  const bool fast = aligned16(w) && aligned16(X) && row_bytes % 16 == 0;
  if (epi.flags() && !fused_route(type, nvec, rows, cols, row_bytes, fast, epi))
    return gemv_unfused(out, w, type, X, nvec, rows, cols, s, epi);
  // Forms with a workspace, which is the caller's (a plan sizes one at instantiation) or a
  // stream-ordered temporary; a call that may not allocate and has no workspace keeps the forms
  // below.
  //  * Q4_K batches of 12-24 vectors or more (many_batch; encoder and prefill sizes): activations
  //    converted once, the weights streamed once per 64 vectors, bit-identical per vector to the
  //    one-vector kernel (k_gemv_q4k_many), with the bias added in its epilogue.
  //  * smaller Q4_K batches (q4s_batch): the K ranges split over workgroups (k_gemv_q4s), bit-identical
  //    per vector to the one-vector kernel, the bias added in its sum launch;
  //  * Q6_K batches (q6_batched): the matrix-core form with the K range split over workgroups
  //    (k_gemv_q6s), bit-identical per vector to the VALU kernel; a bias is added after;
  //  * Q6_K batches with the RMSNorm prologue (q6_norm_batched): the standalone norm into the
  //    workspace, then that form on the normalised activations.
  size_t need = 0;
  if (const WsForm form = ws_route(type, nvec, rows, cols, row_bytes, fast, epi, &need); form != WS_NONE) {
    const bool own = epi.ws && epi.ws_bytes >= need;
    void* ws = own ? epi.ws : epi.no_alloc ? nullptr : gemm_temp_alloc(need, s);
    if (ws) {
      uint32_t* cnt = own && epi.cnt_n >= gemv_q6s_counters(nvec, rows, cols) ? epi.cnt : nullptr;
      bool ok;
      if (form == WS_Q6S_NORM) {  // the normalised activations first, the block sums after them
        const size_t xb = ws_align((size_t)nvec * (size_t)cols * sizeof(float));
        auto* xn = static_cast<float*>(ws);
        launch_rmsnorm(xn, X, epi.norm_w, epi.eps, nvec, cols, s);
        ok = launch_gemv_q6s(w, xn, out, nvec, rows, cols, row_bytes, need > xb ? static_cast<uint8_t*>(ws) + xb : nullptr,
                             s, cnt);
      } else {
        ok = form == WS_MANY ? launch_gemv_q4k_many(w, X, out, epi.bias, nvec, rows, cols, row_bytes, ws, s)
             : form == WS_Q4S ? launch_gemv_q4s(w, X, out, epi.bias, nvec, rows, cols, row_bytes, ws, s)
                              : launch_gemv_q6s(w, X, out, nvec, rows, cols, row_bytes, ws, s, cnt);
      }
      if (!own) gemm_temp_free(ws, s);
      if (!ok) return refused();
      if (form == WS_Q6S && epi.bias) launch_add_bias(out, epi.bias, nvec, rows, s);
      return hip_status();
    }
  }
  if (epi.bias) {  // every other route: the plain product, then the bias add
    GemvEpi plain = epi;
    plain.bias = nullptr;
    if (int rc = gemv(out, w, type, X, nvec, rows, cols, s, plain); rc != QVX_OK) return rc;
    launch_add_bias(out, epi.bias, nvec, rows, s);
    return hip_status();
  }
  // Unquantised weights stream through the float kernel.
  if (fast && (type == T_F32 || type == T_F16 || type == T_BF16) &&
      launch_gemv_float(type, w, X, out, nvec, rows, cols, row_bytes, s))
    return hip_status();
  // The fast kernels take any number of vectors, a few per launch; each vector's arithmetic is the
  // same in every launch, so batches stay bit-identical to single vectors.  Q4_K runs on the matrix
  // cores (up to gemv_mx_max_nv vectors per launch), the other formats on the VALU kernel; shapes
  // neither covers go to the generic kernel.
  // Q4_K batches of two or more vectors, 8 at a time: a chunk of up to 3 vectors (2 on long rows)
  // runs on the one-vector kernel, several vectors a launch (measured faster there); larger chunks
  // take a batched matrix-core form: the one that stages a whole row's activation fragments in LDS
  // where they fit, else the long-row one that converts them per super-block.  All three forms are
  // bit-identical per vector.
  if (fast && type == T_Q4_K && nvec >= 2 && (gemv_mxb_supported(cols) || gemv_mxj_supported(cols))) {
    const bool whole = gemv_mxb_supported(cols) != 0;
    const int small = q4k_small(cols);
    for (int v0 = 0; v0 < nvec; v0 += 8) {
      const int nv = nvec - v0 < 8 ? nvec - v0 : 8;
      const float* Xv = X + (size_t)v0 * cols;
      float* Yv = out + (size_t)v0 * nout;
      const bool ok = nv <= small ? launch_gemv_mx_q4k(w, Xv, Yv, nv, rows, cols, row_bytes, epi, s)
                      : whole     ? launch_gemv_mxb_q4k(w, Xv, Yv, nv, rows, cols, row_bytes, epi, s)
                                  : launch_gemv_mxj_q4k(w, Xv, Yv, nv, rows, cols, row_bytes, s);
      if (!ok) return refused();
    }
    return hip_status();
  }
  // Q6_K batches of rows of one 64-slot block take the matrix-core form here (it needs no
  // workspace); longer rows took it above, or (no workspace) stay on the VALU kernel below.
  if (fast && type == T_Q6_K && q6_batched(nvec, rows, cols) && !epi.flags()) {
    size_t need = 0;
    if (gemv_q6s_route(nvec, rows, cols, row_bytes, &need) && need == 0) {
      if (!launch_gemv_q6s(w, X, out, nvec, rows, cols, row_bytes, nullptr, s, nullptr)) return refused();
      return hip_status();
    }
  }
  const int mx = (fast && type == T_Q4_K) ? gemv_mx_max_nv(cols) : 0;
  if (mx > 0) {
    for (int v0 = 0; v0 < nvec; v0 += mx) {
      const int nv = nvec - v0 < mx ? nvec - v0 : mx;
      if (!launch_gemv_mx_q4k(w, X + (size_t)v0 * cols, out + (size_t)v0 * nout, nv, rows, cols, row_bytes, epi, s))
        return refused();
    }
    return hip_status();
  }
  if (fast && launch_gemv_fast(type, w, X, out, nvec, rows, cols, row_bytes, epi, s)) return hip_status();
  if (epi.flags()) return refused();  // fused_route() promised a fused kernel
  for (int v0 = 0; v0 < nvec; v0 += 16) {
    const int nv = nvec - v0 < 16 ? nvec - v0 : 16;
    if (!launch_gemv_generic(type, w, X + (size_t)v0 * cols, out + (size_t)v0 * rows, rows, cols, nv, row_bytes, s))
      return refused();
  }
  return hip_status();
}

// Makes `dev` current for a scope and restores the caller's device.
struct DeviceGuard {
  int prev = -1;
  bool ok = false;
  explicit DeviceGuard(int dev) {
    if (hipGetDevice(&prev) != hipSuccess) return;
    ok = prev == dev || hipSetDevice(dev) == hipSuccess;
  }
  ~DeviceGuard() {
    int cur = -1;
    if (prev >= 0 && hipGetDevice(&cur) == hipSuccess && cur != prev) (void)hipSetDevice(prev);
  }
};

// Device staging of the synchronous host-pointer entry points: a stream-ordered block of the library's
// memory pool on the null stream (the stream their synchronous copies run on), returned to the pool
// when the call ends.  No per-thread state, so nothing is freed from a thread-exit destructor while
// the HIP runtime may already be tearing down.
struct HostStage {
  void* p = nullptr;
  explicit HostStage(size_t n) : p(gemm_temp_alloc(n, nullptr)) {}
  ~HostStage() { gemm_temp_free(p, nullptr); }
  HostStage(const HostStage&) = delete;
  HostStage& operator=(const HostStage&) = delete;
};

inline size_t align_up(size_t n) { return (n + 255) & ~size_t(255); }

// Device address of this device's copy of `scratch` (below), resolved once per device.
std::mutex g_scratch_mu;
void* g_scratch[kMaxDevices];

// Device address of this device's scratch (the device current at the call), null on failure.
void* scratch_ptr() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return nullptr;
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch[dev]) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) {
      (void)hipGetLastError();
      return nullptr;
    }
    g_scratch[dev] = p;
  }
  return g_scratch[dev];
}

}  // namespace

namespace {

// A fused call in a plan: recorded only when a kernel folds the norm / SwiGLU in, since a replay
// allocates nothing (the unfused route needs pool temporaries).
int plan_add_fused(qvx_plan* plan, float* d_out, const void* d_w, uint32_t type, const float* d_X, int n_vec,
                          int rows, int cols, const GemvEpi& epi) {
  if (!plan) return QVX_E_NULL;
  if (plan->exec) return QVX_E_STATE;
  const TypeInfo* ti = nullptr;
  if (n_vec <= 0) return QVX_E_NVEC;
  if (int rc = check_matmul(type, cols, &ti); rc != QVX_OK) return rc;
  if (rows <= 0) return QVX_OK;
  if (!d_out || (cols > 0 && (!d_w || !d_X))) return QVX_E_NULL;
  if (cols > 0) {
    const size_t row_bytes = (size_t)(cols / (int)ti->block) * ti->bytes;
    const bool fast = aligned16(d_w) && aligned16(d_X) && row_bytes % 16 == 0;
    if (!fused_route(type, n_vec, rows, cols, row_bytes, fast, epi)) return QVX_E_SHAPE;
  }
  plan->calls.push_back({d_out, d_w, type, d_X, n_vec, rows, cols, plan->open_group, epi});
  return QVX_OK;
}

}  // namespace

#pragma GCC visibility push(default)
extern "C" {

const char* qvx_version(void) { return "qvx 0.1 gfx950"; }

const char* qvx_strerror(int code) {
  switch (code) {
    case QVX_OK: return "ok";
    case QVX_E_TYPE: return "unsupported ggml type";
    case QVX_E_SHAPE: return "cols is not a whole number of blocks (or bad shape)";
    case QVX_E_NVEC: return "n_vec must be positive";
    case QVX_E_NULL: return "null pointer argument";
    case QVX_E_HIP: return "HIP runtime error";
    case QVX_E_VARIANT: return "unknown GEMM variant";
    case QVX_E_RANGE: return "index or size out of range";
    case QVX_E_STATE: return "plan not instantiated, or changed after instantiation";
    case QVX_E_FORMAT: return "malformed GGUF data";
    case QVX_E_IO: return "file could not be opened or mapped";
    case QVX_E_LIB: return "a runtime library the call needs is missing or failed";
    default: return "unknown qvx status";
  }
}

int qvx_supports(uint32_t type) { return type_info(type) && can_dequantize(type) && gemv_supports(type); }

int qvx_can_dequantize(uint32_t type) { return can_dequantize(type) ? 1 : 0; }

int qvx_type_traits(uint32_t type, uint32_t* block_size, uint32_t* type_size) {
  const TypeInfo* t = type_info(type);
  if (!t) return 0;
  if (block_size) *block_size = t->block;
  if (type_size) *type_size = t->bytes;
  return 1;
}

float qvx_fp16_to_float(uint16_t h) { return f16_bits_to_f32(h); }

float qvx_bf16_to_float(uint16_t b) { return __builtin_bit_cast(float, (uint32_t)b << 16); }

int qvx_qmatmul(float* d_out, const void* d_w, uint32_t type, const float* d_x, int rows, int cols, void* stream) {
  return gemv(d_out, d_w, type, d_x, 1, rows, cols, as_stream(stream));
}

int qvx_qmatmul_n(float* d_out, const void* d_w, uint32_t type, const float* d_X, int n_vec, int rows, int cols,
                  void* stream) {
  return gemv(d_out, d_w, type, d_X, n_vec, rows, cols, as_stream(stream));
}

// Checks a grouped call's members as qvx_qmatmul checks each one and collects those with rows into
// m (at most QVX_GROUP_MAX); *k = their count.
static int group_members(float* const* d_out, const void* const* d_w, const uint32_t* types, const int* rows, int n,
                         const float* d_x, int cols, GemvMember* m, int* k) {
  if (n < 1 || n > QVX_GROUP_MAX) return QVX_E_NVEC;
  if (!d_out || !d_w || !types || !rows) return QVX_E_NULL;
  *k = 0;
  for (int i = 0; i < n; ++i) {
    const TypeInfo* ti = nullptr;
    if (int rc = check_matmul(types[i], cols, &ti); rc != QVX_OK) return rc;
    if (rows[i] <= 0) continue;  // nothing to compute, as for qvx_qmatmul
    if (!d_out[i] || (cols > 0 && (!d_w[i] || !d_x))) return QVX_E_NULL;
    const size_t row_bytes = cols > 0 ? (size_t)(cols / (int)ti->block) * ti->bytes : 0;
    m[(*k)++] = GemvMember{d_w[i], d_out[i], types[i], rows[i], row_bytes};
  }
  return QVX_OK;
}

// One launch for the members when the grouped kernel takes them all, else one qmatmul (or
// qmatmul_n_rmsnorm) each.
static int gemv_group(const GemvMember* m, int k, const float* x, int cols, const GemvEpi& epi, hipStream_t s) {
  bool fast = cols > 0 && aligned16(x);
  for (int i = 0; i < k; ++i) fast = fast && aligned16(m[i].w) && m[i].row_bytes % 16 == 0;
  if (fast && launch_gemv_group(m, k, x, cols, epi, s)) return hip_status();
  for (int i = 0; i < k; ++i)
    if (int rc = gemv(m[i].y, m[i].w, m[i].type, x, 1, m[i].rows, cols, s, epi); rc != QVX_OK) return rc;
  return QVX_OK;
}

int qvx_qmatmul_group(float* const* d_out, const void* const* d_w, const uint32_t* types, const int* rows, int n,
                      const float* d_x, const float* d_norm_w, float eps, int cols, void* stream) {
  GemvMember m[QVX_GROUP_MAX];
  int k = 0;
  if (int rc = group_members(d_out, d_w, types, rows, n, d_x, cols, m, &k); rc != QVX_OK) return rc;
  GemvEpi epi;
  epi.norm_w = d_norm_w;
  epi.eps = eps;
  return k ? gemv_group(m, k, d_x, cols, epi, as_stream(stream)) : QVX_OK;
}

int qvx_qmatmul_n_bias(float* d_out, const void* d_w, uint32_t type, const float* d_X, const float* d_bias,
                       int n_vec, int rows, int cols, void* stream) {
  GemvEpi epi;
  epi.bias = d_bias;
  return gemv(d_out, d_w, type, d_X, n_vec, rows, cols, as_stream(stream), epi);
}

int qvx_qmatmul_n_rmsnorm(float* d_out, const void* d_w, uint32_t type, const float* d_X, const float* d_norm_w,
                          float eps, int n_vec, int rows, int cols, void* stream) {
  const TypeInfo* ti = nullptr;
  if (n_vec <= 0) return QVX_E_NVEC;
  if (int rc = check_matmul(type, cols, &ti); rc != QVX_OK) return rc;
  if (rows > 0 && cols > 0 && !d_norm_w) return QVX_E_NULL;
  GemvEpi epi;
  epi.norm_w = d_norm_w;
  epi.eps = eps;
  return gemv(d_out, d_w, type, d_X, n_vec, rows, cols, as_stream(stream), epi);
}

int qvx_qmatmul_swiglu(float* d_out, const void* d_w_gu, uint32_t type, const float* d_X, const float* d_norm_w,
                       float eps, int n_vec, int ffn, int cols, void* stream) {
  const TypeInfo* ti = nullptr;
  if (n_vec <= 0) return QVX_E_NVEC;
  if (int rc = check_matmul(type, cols, &ti); rc != QVX_OK) return rc;
  if (ffn < 0 || ffn % 16 != 0) return QVX_E_SHAPE;
  if (ffn > (1 << 30)) return QVX_E_RANGE;
  GemvEpi epi;
  epi.norm_w = d_norm_w;
  epi.eps = eps;
  epi.swiglu = true;
  return gemv(d_out, d_w_gu, type, d_X, n_vec, 2 * ffn, cols, as_stream(stream), epi);
}

int qvx_rmsnorm(float* d_out, const float* d_x, const float* d_w, float eps, int n_vec, int n, void* stream) {
  if (n_vec <= 0) return QVX_E_NVEC;
  if (n < 0 || n > kNormChunk * kNormMaxChunks) return QVX_E_RANGE;
  if (n == 0) return QVX_OK;
  if (!d_out || !d_x || !d_w) return QVX_E_NULL;
  launch_rmsnorm(d_out, d_x, d_w, eps, n_vec, n, as_stream(stream));
  return hip_status();
}

int qvx_swiglu(float* d_out, const float* d_gate, const float* d_up, size_t n, void* stream) {
  if (n == 0) return QVX_OK;
  if (!d_out || !d_gate || !d_up) return QVX_E_NULL;
  launch_swiglu(d_out, d_gate, d_up, n, as_stream(stream));
  return hip_status();
}

int qvx_interleave_rows16(void* d_dst, const void* d_a, const void* d_b, uint32_t type, int rows, int cols,
                          void* stream) {
  const TypeInfo* t = type_info(type);
  if (!t) return QVX_E_TYPE;
  if (t->block == 0 || cols < 0 || cols % (int)t->block != 0 || rows < 0 || rows % 16 != 0) return QVX_E_SHAPE;
  if (rows == 0 || cols == 0) return QVX_OK;
  if (!d_dst || !d_a || !d_b) return QVX_E_NULL;
  const size_t g = 16 * (size_t)(cols / (int)t->block) * t->bytes;  // bytes of 16 rows
  const hipStream_t s = as_stream(stream);
  auto* dst = static_cast<uint8_t*>(d_dst);
  if (hipMemcpy2DAsync(dst, 2 * g, d_a, g, g, (size_t)rows / 16, hipMemcpyDeviceToDevice, s) != hipSuccess ||
      hipMemcpy2DAsync(dst + g, 2 * g, d_b, g, g, (size_t)rows / 16, hipMemcpyDeviceToDevice, s) != hipSuccess) {
    (void)hipGetLastError();
    return QVX_E_HIP;
  }
  return hip_status();
}

int qvx_dequantize(uint32_t type, const void* d_src, float* d_dst, size_t n, void* stream) {
  const TypeInfo* t = type_info(type);
  if (!t || !can_dequantize(type)) return QVX_E_TYPE;
  // The reference converts n / blockSize whole blocks and leaves dst[n - n % blockSize, n) as it was
  // (dequant.cpp:38-210: every block loop runs to n / QK); the same here.
  n -= n % t->block;
  if (n == 0) return QVX_OK;
  if (!d_src || !d_dst) return QVX_E_NULL;
  if (!launch_dequant(type, d_src, d_dst, n, as_stream(stream))) return QVX_E_HIP;
  return hip_status();
}

int qvx_dequant_row(const void* d_w, uint32_t type, int cols, int row, float* d_dst, void* stream) {
  const TypeInfo* t = type_info(type);
  if (!t || !can_dequantize(type)) return QVX_E_TYPE;
  if (t->block == 0 || cols % (int)t->block != 0) return QVX_E_SHAPE;
  if (row < 0 || cols < 0) return QVX_E_RANGE;
  if (cols == 0) return QVX_OK;
  if (!d_w || !d_dst) return QVX_E_NULL;
  const size_t row_bytes = (size_t)(cols / (int)t->block) * t->bytes;
  const auto* src = static_cast<const uint8_t*>(d_w) + (size_t)row * row_bytes;
  if (!launch_dequant(type, src, d_dst, (size_t)cols, as_stream(stream))) return QVX_E_HIP;
  return hip_status();
}

int qvx_qgemm_f16(float* d_out, const void* d_w, uint32_t type, const uint16_t* d_X, int M, int rows, int cols,
                  int variant, void* stream) {
  const TypeInfo* ti = nullptr;
  if (M <= 0) return QVX_E_NVEC;
  if (variant != QVX_GEMM_BF16 && variant != QVX_GEMM_I8 && variant != QVX_GEMM_F16) return QVX_E_VARIANT;
  if (int rc = check_matmul(type, cols, &ti); rc != QVX_OK) return rc;
  if (variant == QVX_GEMM_I8 && type != T_Q4_K) return QVX_E_TYPE;
  if (rows <= 0) return QVX_OK;
  if (!d_out) return QVX_E_NULL;
  if (cols <= 0) {
    launch_zero(d_out, (size_t)rows * (size_t)M, as_stream(stream));
    return hip_status();
  }
  if (!d_w || !d_X) return QVX_E_NULL;
  const int rc = launch_qgemm(d_out, d_w, type, d_X, M, rows, cols, variant, as_stream(stream), nullptr, 0);
  if (rc != QVX_OK) return rc;
  return hip_status();
}

int qvx_qgemm_plan_q4k(int M, int rows, int cols, int cus, int* desc, int cap) {
  if (M <= 0 || rows <= 0 || cols <= 0 || cols % 256) return QVX_E_SHAPE;
  if (!desc && cap > 0) return QVX_E_NULL;
  return q4k_plan_desc(M, rows, cols, cus, desc, cap);
}

int qvx_qgemm_f16_noalloc(float* d_out, const void* d_w, uint32_t type, const uint16_t* d_X, int M, int rows,
                          int cols, int variant, void* stream) {
  const TypeInfo* ti = nullptr;
  if (M <= 0) return QVX_E_NVEC;
  if (variant != QVX_GEMM_BF16 && variant != QVX_GEMM_I8 && variant != QVX_GEMM_F16) return QVX_E_VARIANT;
  if (int rc = check_matmul(type, cols, &ti); rc != QVX_OK) return rc;
  if (variant == QVX_GEMM_I8 && type != T_Q4_K) return QVX_E_TYPE;
  if (rows <= 0) return QVX_OK;
  if (!d_out) return QVX_E_NULL;
  if (cols <= 0) {
    launch_zero(d_out, (size_t)rows * (size_t)M, as_stream(stream));
    return hip_status();
  }
  if (!d_w || !d_X) return QVX_E_NULL;
  void* ws = scratch_ptr();
  if (!ws) return QVX_E_HIP;
  const int rc = launch_qgemm(d_out, d_w, type, d_X, M, rows, cols, variant, as_stream(stream), ws, kScratchBytes);
  if (rc != QVX_OK) return rc;
  return hip_status();
}

int qvx_gemm16(float* d_out, const uint16_t* d_X, const uint16_t* d_B, int M, int N, int K, int variant,
               void* stream) {
  if (variant != QVX_GEMM_BF16 && variant != QVX_GEMM_F16) return QVX_E_VARIANT;
  if (M < 0 || N < 0 || K < 0) return QVX_E_SHAPE;
  if (M == 0 || N == 0) return QVX_OK;
  if (!d_out) return QVX_E_NULL;
  if (K == 0) {
    launch_zero(d_out, (size_t)M * (size_t)N, as_stream(stream));
    return hip_status();
  }
  if (!d_X || !d_B) return QVX_E_NULL;
  const int rc = launch_gemm16_entry(d_out, d_X, d_B, M, N, K, variant == QVX_GEMM_BF16, as_stream(stream));
  if (rc != QVX_OK) return rc;
  return hip_status();
}

int qvx_dequantize16(uint32_t type, const void* d_src, uint16_t* d_dst, size_t n, int bf16, void* stream) {
  const TypeInfo* t = type_info(type);
  if (!t || !can_dequantize(type)) return QVX_E_TYPE;
  n -= n % t->block;  // whole blocks, as qvx_dequantize
  if (n == 0) return QVX_OK;
  if (!d_src || !d_dst) return QVX_E_NULL;
  if (!launch_dequant16(type, d_src, d_dst, n, bf16 != 0, as_stream(stream))) return QVX_E_HIP;
  return hip_status();
}

int qvx_quantize_act_q8(const uint16_t* d_X, int M, int K, int8_t* d_q, float* d_scale, int32_t* d_qsum,
                        void* stream) {
  if (M <= 0 || K <= 0 || K % 32 != 0) return QVX_E_SHAPE;
  if (!d_X || !d_q || !d_scale || !d_qsum) return QVX_E_NULL;
  const int rc = launch_quantize_act_q8(d_X, M, K, d_q, d_scale, d_qsum, as_stream(stream));
  if (rc != QVX_OK) return rc;
  return hip_status();
}

int qvx_fill_synthetic(void* d_w, uint32_t type, int rows, int cols, uint64_t seed, float scale_mul, void* stream) {
  const TypeInfo* t = type_info(type);
  if (!t || (type != T_Q8_0 && type != T_Q4_0 && type != T_Q4_K && type != T_Q5_K &&
              type != T_Q6_K)) return QVX_E_TYPE;
  if (rows < 0 || cols < 0 || cols % (int)t->block != 0) return QVX_E_SHAPE;
  if (!d_w) return QVX_E_NULL;
  const size_t nblk = (size_t)rows * (size_t)(cols / (int)t->block);
  if (!launch_fill_synthetic(d_w, type, nblk, seed, scale_mul, as_stream(stream))) return QVX_E_TYPE;
  return hip_status();
}

int qvx_fill_normal_f32(float* d_x, size_t n, uint64_t seed, float mul, void* stream) {
  if (n && !d_x) return QVX_E_NULL;
  launch_fill_normal_f32(d_x, n, seed, mul, as_stream(stream));
  return hip_status();
}

int qvx_fill_normal_f16(uint16_t* d_x, size_t n, uint64_t seed, float mul, void* stream) {
  if (n && !d_x) return QVX_E_NULL;
  launch_fill_normal_f16(d_x, n, seed, mul, as_stream(stream));
  return hip_status();
}

int qvx_bench_read(const void* d_src, size_t n, uint32_t* d_flag, void* stream) {
  if (n % 16 != 0) return QVX_E_RANGE;
  if (n && (!d_src || !d_flag)) return QVX_E_NULL;
  if (reinterpret_cast<uintptr_t>(d_src) & 15u) return QVX_E_RANGE;
  launch_read16(d_src, n / 16, d_flag, as_stream(stream));
  return hip_status();
}

// ---- plans ---------------------------------------------------------------------------------------

int qvx_plan_create(qvx_plan** plan) {
  if (!plan) return QVX_E_NULL;
  *plan = nullptr;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return QVX_E_HIP;
  auto* p = new (std::nothrow) qvx_plan;
  if (!p) return QVX_E_HIP;
  p->device = dev;
  *plan = p;
  return QVX_OK;
}

int qvx_plan_add_qmatmul_n(qvx_plan* plan, float* d_out, const void* d_w, uint32_t type, const float* d_X,
                           int n_vec, int rows, int cols) {
  if (!plan) return QVX_E_NULL;
  if (plan->exec) return QVX_E_STATE;
  const TypeInfo* ti = nullptr;
  if (n_vec <= 0) return QVX_E_NVEC;
  if (int rc = check_matmul(type, cols, &ti); rc != QVX_OK) return rc;
  if (rows <= 0) return QVX_OK;
  if (!d_out || (cols > 0 && (!d_w || !d_X))) return QVX_E_NULL;
  plan->calls.push_back({d_out, d_w, type, d_X, n_vec, rows, cols, plan->open_group, GemvEpi{}});
  return QVX_OK;
}

// One recorded call: a grouped call or a plain / fused GEMV.
static int run_call(const qvx_plan& plan, const qvx_plan::Call& c, hipStream_t s) {
  if (!c.members.empty()) return gemv_group(c.members.data(), (int)c.members.size(), c.X, c.cols, c.epi, s);
  GemvEpi epi = c.epi;
  epi.no_alloc = true;  // a captured call may not allocate
  if (plan.ws && c.ws_bytes) {
    epi.ws = static_cast<uint8_t*>(plan.ws) + c.ws_off;
    epi.ws_bytes = c.ws_bytes;
  }
  if (plan.ws && c.cnt_n) {
    epi.cnt = reinterpret_cast<uint32_t*>(static_cast<uint8_t*>(plan.ws) + c.cnt_off);
    epi.cnt_n = c.cnt_n;
  }
  return gemv(c.out, c.w, c.type, c.X, c.nvec, c.rows, c.cols, s, epi);
}

// Lays out the plan's workspace: each call whose form takes a workspace gets a 256-byte aligned
// slice; calls in order share offset 0, the calls of one fork (which run concurrently) get disjoint
// slices.  After them, each call that can use tile counters gets its own slice of them (zeroed by
// qvx_plan_instantiate; the kernels leave them zero, so no other data may share them).  Returns the
// bytes the plan needs.
static size_t plan_ws_layout(qvx_plan& plan) {
  size_t total = 0;
  for (size_t i = 0; i < plan.calls.size();) {
    const int g = plan.calls[i].group;
    size_t n = 1;
    while (g >= 0 && i + n < plan.calls.size() && plan.calls[i + n].group == g) ++n;
    size_t off = 0;
    for (size_t k = i; k < i + n; ++k) {
      auto& c = plan.calls[k];
      c.ws_off = c.ws_bytes = 0;
      c.cnt_off = 0;
      c.cnt_n = 0;
      if (!c.members.empty() || c.cols <= 0 || c.rows <= 0) continue;
      const TypeInfo* ti = type_info(c.type);
      if (!ti || ti->block == 0) continue;
      const size_t row_bytes = (size_t)(c.cols / (int)ti->block) * ti->bytes;
      const bool fast = aligned16(c.w) && aligned16(c.X) && row_bytes % 16 == 0;
      size_t need = 0;
      const WsForm form = ws_route(c.type, c.nvec, c.rows, c.cols, row_bytes, fast, c.epi, &need);
      if (form == WS_NONE) continue;
      c.ws_off = off;
      c.ws_bytes = need;
      off += (need + 255) & ~(size_t)255;
      if (form == WS_Q6S || form == WS_Q6S_NORM) c.cnt_n = gemv_q6s_counters(c.nvec, c.rows, c.cols);
    }
    if (off > total) total = off;
    i += n;
  }
  for (auto& c : plan.calls) {
    if (!c.cnt_n) continue;
    c.cnt_off = total;
    total += ((size_t)c.cnt_n * 4 + 255) & ~(size_t)255;
  }
  return total;
}

int qvx_plan_add_qmatmul_group(qvx_plan* plan, float* const* d_out, const void* const* d_w, const uint32_t* types,
                               const int* rows, int n, const float* d_x, const float* d_norm_w, float eps,
                               int cols) {
  if (!plan) return QVX_E_NULL;
  if (plan->exec) return QVX_E_STATE;
  GemvMember m[QVX_GROUP_MAX];
  int k = 0;
  if (int rc = group_members(d_out, d_w, types, rows, n, d_x, cols, m, &k); rc != QVX_OK) return rc;
  if (k == 0) return QVX_OK;
  GemvEpi epi;
  epi.norm_w = d_norm_w;
  epi.eps = eps;
  if (d_norm_w && cols > 0)  // a replay allocates nothing: every member must take the folded norm
    for (int i = 0; i < k; ++i)
      if (!fused_route(m[i].type, 1, m[i].rows, cols, m[i].row_bytes,
                       aligned16(m[i].w) && aligned16(d_x) && m[i].row_bytes % 16 == 0, epi))
        return QVX_E_SHAPE;
  qvx_plan::Call c{nullptr, nullptr, 0, d_x, 1, 0, cols, plan->open_group, epi, {}};
  c.members.assign(m, m + k);
  plan->calls.push_back(std::move(c));
  return QVX_OK;
}

int qvx_plan_add_qmatmul_n_rmsnorm(qvx_plan* plan, float* d_out, const void* d_w, uint32_t type, const float* d_X,
                                   const float* d_norm_w, float eps, int n_vec, int rows, int cols) {
  if (plan && !d_norm_w && n_vec > 0 && rows > 0 && cols > 0) return QVX_E_NULL;
  GemvEpi epi;
  epi.norm_w = d_norm_w;
  epi.eps = eps;
  return plan_add_fused(plan, d_out, d_w, type, d_X, n_vec, rows, cols, epi);
}

int qvx_plan_add_qmatmul_swiglu(qvx_plan* plan, float* d_out, const void* d_w_gu, uint32_t type, const float* d_X,
                                const float* d_norm_w, float eps, int n_vec, int ffn, int cols) {
  if (ffn < 0 || ffn % 16 != 0) return QVX_E_SHAPE;
  if (ffn > (1 << 30)) return QVX_E_RANGE;
  GemvEpi epi;
  epi.norm_w = d_norm_w;
  epi.eps = eps;
  epi.swiglu = true;
  return plan_add_fused(plan, d_out, d_w_gu, type, d_X, n_vec, 2 * ffn, cols, epi);
}

int qvx_plan_fork(qvx_plan* plan) {
  if (!plan) return QVX_E_NULL;
  if (plan->exec || plan->open_group >= 0) return QVX_E_STATE;
  plan->open_group = plan->groups++;
  return QVX_OK;
}

int qvx_plan_join(qvx_plan* plan) {
  if (!plan) return QVX_E_NULL;
  if (plan->exec || plan->open_group < 0) return QVX_E_STATE;
  plan->open_group = -1;
  return QVX_OK;
}

int qvx_plan_size(const qvx_plan* plan) { return plan ? (int)plan->calls.size() : 0; }

int qvx_plan_run_eager(const qvx_plan* plan, void* stream) {
  if (!plan) return QVX_E_NULL;
  for (const auto& c : plan->calls)
    if (int rc = run_call(*plan, c, as_stream(stream)); rc != QVX_OK) return rc;
  return QVX_OK;
}

// Records the plan's calls on `cs` (which is capturing).  A group of n independent calls gets
// n branches: the first on `cs`, the others on side streams that wait for the fork point and are
// joined back into `cs` after the group.
static int plan_record(const qvx_plan* plan, hipStream_t cs, std::vector<hipStream_t>& side,
                       std::vector<hipEvent_t>& events) {
  const auto& calls = plan->calls;
  auto event = [&](hipEvent_t* e) {
    if (hipEventCreateWithFlags(e, hipEventDisableTiming) != hipSuccess) return false;
    events.push_back(*e);
    return true;
  };
  for (size_t i = 0; i < calls.size();) {
    const int g = calls[i].group;
    size_t n = 1;
    while (g >= 0 && i + n < calls.size() && calls[i + n].group == g) ++n;
    if (n == 1) {
      const auto& c = calls[i];
      if (int rc = run_call(*plan, c, cs); rc != QVX_OK) return rc;
      ++i;
      continue;
    }
    while (side.size() < n - 1) {
      hipStream_t st = nullptr;
      if (hipStreamCreateWithFlags(&st, hipStreamNonBlocking) != hipSuccess) return QVX_E_HIP;
      side.push_back(st);
    }
    hipEvent_t fork = nullptr;
    if (!event(&fork) || hipEventRecord(fork, cs) != hipSuccess) return QVX_E_HIP;
    for (size_t k = 0; k < n; ++k) {
      const auto& c = calls[i + k];
      hipStream_t st = k == 0 ? cs : side[k - 1];
      if (k > 0 && hipStreamWaitEvent(st, fork, 0) != hipSuccess) return QVX_E_HIP;
      if (int rc = run_call(*plan, c, st); rc != QVX_OK) return rc;
    }
    for (size_t k = 1; k < n; ++k) {
      hipEvent_t done = nullptr;
      if (!event(&done) || hipEventRecord(done, side[k - 1]) != hipSuccess ||
          hipStreamWaitEvent(cs, done, 0) != hipSuccess)
        return QVX_E_HIP;
    }
    i += n;
  }
  return QVX_OK;
}

int qvx_plan_instantiate(qvx_plan* plan) {
  if (!plan) return QVX_E_NULL;
  if (plan->exec) return QVX_OK;
  plan->open_group = -1;
  DeviceGuard guard(plan->device);
  if (!guard.ok) return QVX_E_HIP;
  if (const size_t wsb = plan_ws_layout(*plan)) {
    if (hipMalloc(&plan->ws, wsb) != hipSuccess) {
      plan->ws = nullptr;
      (void)hipGetLastError();
      return QVX_E_HIP;
    }
    if (hipMemset(plan->ws, 0, wsb) != hipSuccess) {  // the counters start at zero (outside any capture)
      (void)hipFree(plan->ws);
      plan->ws = nullptr;
      (void)hipGetLastError();
      return QVX_E_HIP;
    }
  }
  // Capture on streams of the plan's own (default priority), in thread-local mode: the GEMV
  // launches make no calls that capture forbids.
  hipStream_t cs = nullptr;
  if (hipStreamCreateWithFlags(&cs, hipStreamNonBlocking) != hipSuccess) return QVX_E_HIP;
  std::vector<hipStream_t> side;
  std::vector<hipEvent_t> events;
  int rc = QVX_OK;
  hipGraph_t graph = nullptr;
  if (hipStreamBeginCapture(cs, hipStreamCaptureModeThreadLocal) != hipSuccess) {
    rc = QVX_E_HIP;
  } else {
    rc = plan_record(plan, cs, side, events);
    if (hipStreamEndCapture(cs, &graph) != hipSuccess && rc == QVX_OK) rc = QVX_E_HIP;
  }
  hipGraphExec_t exec = nullptr;
  if (rc == QVX_OK && hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0) != hipSuccess) rc = QVX_E_HIP;
  for (hipEvent_t e : events) (void)hipEventDestroy(e);
  for (hipStream_t st : side) (void)hipStreamDestroy(st);
  (void)hipStreamDestroy(cs);
  if (rc != QVX_OK) {
    if (graph) (void)hipGraphDestroy(graph);
    if (plan->ws) (void)hipFree(plan->ws);
    plan->ws = nullptr;
    (void)hipGetLastError();
    return rc;
  }
  plan->graph = graph;
  plan->exec = exec;
  return QVX_OK;
}

int qvx_plan_launch(qvx_plan* plan, void* stream) {
  if (!plan) return QVX_E_NULL;
  if (!plan->exec) return QVX_E_STATE;
  if (hipGraphLaunch(plan->exec, as_stream(stream)) != hipSuccess) return QVX_E_HIP;
  return QVX_OK;
}

void qvx_plan_destroy(qvx_plan* plan) {
  if (!plan) return;
  {
    DeviceGuard guard(plan->device);
    if (plan->exec) (void)hipGraphExecDestroy(plan->exec);
    if (plan->graph) (void)hipGraphDestroy(plan->graph);
    if (plan->ws) (void)hipFree(plan->ws);
  }
  delete plan;
}

// ---- synchronous host-pointer forms --------------------------------------------------------------

int qvx_qmatmul_n_host(float* out, const void* w, uint32_t type, const float* X, int n_vec, int rows, int cols) {
  const TypeInfo* ti = nullptr;
  if (n_vec <= 0) return QVX_E_NVEC;
  if (int rc = check_matmul(type, cols, &ti); rc != QVX_OK) return rc;
  if (rows <= 0) return QVX_OK;
  if (!out) return QVX_E_NULL;
  if (cols <= 0) {
    std::memset(out, 0, sizeof(float) * (size_t)rows * (size_t)n_vec);
    return QVX_OK;
  }
  if (!w || !X) return QVX_E_NULL;
  const size_t wb = (size_t)rows * (size_t)(cols / (int)ti->block) * ti->bytes;
  const size_t xb = sizeof(float) * (size_t)n_vec * (size_t)cols;
  const size_t ob = sizeof(float) * (size_t)n_vec * (size_t)rows;
  HostStage stage(align_up(wb) + align_up(xb) + align_up(ob));
  auto* base = static_cast<uint8_t*>(stage.p);
  if (!base) return QVX_E_HIP;
  void* dw = base;
  auto* dx = reinterpret_cast<float*>(base + align_up(wb));
  auto* dout = reinterpret_cast<float*>(base + align_up(wb) + align_up(xb));
  if (hipMemcpy(dw, w, wb, hipMemcpyHostToDevice) != hipSuccess) return hip_status();
  if (hipMemcpy(dx, X, xb, hipMemcpyHostToDevice) != hipSuccess) return hip_status();
  const int rc = gemv(dout, dw, type, dx, n_vec, rows, cols, nullptr);
  if (rc != QVX_OK) return rc;
  if (hipMemcpy(out, dout, ob, hipMemcpyDeviceToHost) != hipSuccess) return hip_status();
  return QVX_OK;
}

int qvx_qmatmul_host(float* out, const void* w, uint32_t type, const float* x, int rows, int cols) {
  return qvx_qmatmul_n_host(out, w, type, x, 1, rows, cols);
}

int qvx_dequantize_host(uint32_t type, const void* src, float* dst, size_t n) {
  const TypeInfo* t = type_info(type);
  if (!t || !can_dequantize(type)) return QVX_E_TYPE;
  n -= n % t->block;  // whole blocks only, as qvx_dequantize
  if (n == 0) return QVX_OK;
  if (!src || !dst) return QVX_E_NULL;
  const size_t sb = n / t->block * t->bytes, db = n * sizeof(float);
  HostStage stage(align_up(sb) + align_up(db));
  auto* base = static_cast<uint8_t*>(stage.p);
  if (!base) return QVX_E_HIP;
  auto* ddst = reinterpret_cast<float*>(base + align_up(sb));
  if (hipMemcpy(base, src, sb, hipMemcpyHostToDevice) != hipSuccess) return hip_status();
  if (!launch_dequant(type, base, ddst, n, nullptr)) return QVX_E_HIP;
  if (int rc = hip_status(); rc != QVX_OK) return rc;
  if (hipMemcpy(dst, ddst, db, hipMemcpyDeviceToHost) != hipSuccess) return hip_status();
  return QVX_OK;
}

int qvx_dequant_row_host(const void* w, uint32_t type, int cols, int row, float* dst) {
  const TypeInfo* t = type_info(type);
  if (!t || !can_dequantize(type)) return QVX_E_TYPE;
  if (t->block == 0 || cols % (int)t->block != 0) return QVX_E_SHAPE;
  if (row < 0 || cols < 0) return QVX_E_RANGE;
  if (cols == 0) return QVX_OK;
  if (!w || !dst) return QVX_E_NULL;
  const size_t row_bytes = (size_t)(cols / (int)t->block) * t->bytes;
  return qvx_dequantize_host(type, static_cast<const uint8_t*>(w) + (size_t)row * row_bytes, dst, (size_t)cols);
}

}  // extern "C"
#pragma GCC visibility pop
