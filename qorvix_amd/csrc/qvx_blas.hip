// qvx_blas.hip -- prefill GEMM for the weight types without a hand-written GEMM kernel.
//
// out[m, r] = sum_k X[m, k] * dequant(W)[r, k] for every type qvx_qmatmul accepts other than Q4_K
// (which has its own MFMA kernels): the weight is dequantised into a stream-ordered 16-bit temporary
// (fp16, or bf16 for the bf16 variant, one rounding of the reference's fp32 dequant value), and one
// plain library GEMM multiplies it with X (fp16, or X rounded to bf16), fp32 accumulate and output.
// The reference has no prefill GEMM (it prefills token by token); the semantics are qmatmulN's
// (runtime/src/qmatmul.cpp:64-115) with X converted fp16 -> fp32 exactly.
//
// rocBLAS is loaded with dlopen on the first such call, so the engine carries no link dependency on
// it and callers that never run these GEMMs never load it.  Each host thread keeps one rocBLAS
// handle per device (handles are not safe across threads); the handle is bound to the caller's
// stream for each call.  The first call on a thread and device creates the handle, which allocates,
// so these GEMMs are not for HIP graph capture.
#include "qvx_common.hpp"

#include <dlfcn.h>
#include <rocblas/rocblas.h>

#include <mutex>

namespace qvx {

bool launch_dequant16(uint32_t t, const void* src, uint16_t* dst, size_t n, bool bf16, hipStream_t s);
void* gemm_temp_alloc(size_t bytes, hipStream_t s);
void gemm_temp_free(void* p, hipStream_t s);

namespace {

struct Blas {
  decltype(&rocblas_create_handle) create = nullptr;
  decltype(&rocblas_set_stream) set_stream = nullptr;
  decltype(&rocblas_gemm_ex) gemm_ex = nullptr;
  bool ok = false;
};

const Blas& blas() {
  static Blas b;
  static std::once_flag once;
  std::call_once(once, [] {
    void* h = dlopen("librocblas.so.5", RTLD_NOW | RTLD_LOCAL);
    if (!h) h = dlopen("librocblas.so", RTLD_NOW | RTLD_LOCAL);
    if (!h) return;
    b.create = reinterpret_cast<decltype(b.create)>(dlsym(h, "rocblas_create_handle"));
    b.set_stream = reinterpret_cast<decltype(b.set_stream)>(dlsym(h, "rocblas_set_stream"));
    b.gemm_ex = reinterpret_cast<decltype(b.gemm_ex)>(dlsym(h, "rocblas_gemm_ex"));
    b.ok = b.create && b.set_stream && b.gemm_ex;
  });
  return b;
}

// This thread's handle for device `dev` (nullptr when it cannot be created).  Handles are kept for
// the life of the process: destroying them from thread-exit destructors would race the HIP
// runtime's own teardown at process exit.
rocblas_handle thread_handle(const Blas& b, int dev) {
  thread_local rocblas_handle handles[kMaxDevices] = {};
  if (!handles[dev] && b.create(&handles[dev]) != rocblas_status_success) handles[dev] = nullptr;
  return handles[dev];
}

__global__ __launch_bounds__(256) void k_f16_to_bf16_any(const uint16_t* __restrict__ x, uint16_t* __restrict__ y,
                                                         size_t n) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  const float f = (float)__builtin_bit_cast(_Float16, x[i]);
  const uint32_t u = __builtin_bit_cast(uint32_t, f);  // fp16 -> fp32 is exact; one rounding to bf16
  y[i] = (u & 0x7FFFFFFFu) > 0x7F800000u ? (uint16_t)((u >> 16) | 0x0040u)
                                         : (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

}  // namespace

// Returns 0, or -1 (type not dequantisable), -5 (allocation / HIP), -7 (size beyond the library's
// 32-bit dimensions), -11 (rocBLAS missing or failing).  bf16: the bf16 variant.
int launch_qgemm_dequant(float* out, const void* w, uint32_t t, const uint16_t* X, int M, int rows, int cols,
                         bool bf16, hipStream_t s) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return -5;
  const Blas& b = blas();
  if (!b.ok) return -11;
  rocblas_handle h = thread_handle(b, dev);
  if (!h) return -11;
  const size_t nw = (size_t)rows * (size_t)cols, nx = (size_t)M * (size_t)cols;
  uint16_t* wd = static_cast<uint16_t*>(gemm_temp_alloc(nw * 2u + (bf16 ? nx * 2u : 0u), s));
  if (!wd) return -5;
  if (!launch_dequant16(t, w, wd, nw, bf16, s)) {
    gemm_temp_free(wd, s);
    return -1;
  }
  const uint16_t* xb = X;
  if (bf16) {
    uint16_t* xc = wd + nw;
    k_f16_to_bf16_any<<<(unsigned)((nx + 255) / 256), 256, 0, s>>>(X, xc, nx);
    xb = xc;
  }
  // Column-major view: out^T [rows, M] = W_deq [cols, rows]^T * X [cols, M].
  const rocblas_datatype in = bf16 ? rocblas_datatype_bf16_r : rocblas_datatype_f16_r;
  const float alpha = 1.0f, beta = 0.0f;
  int rc = 0;
  if (b.set_stream(h, s) != rocblas_status_success ||
      b.gemm_ex(h, rocblas_operation_transpose, rocblas_operation_none, rows, M, cols, &alpha, wd, in, cols, xb, in,
                cols, &beta, out, rocblas_datatype_f32_r, rows, out, rocblas_datatype_f32_r, rows,
                rocblas_datatype_f32_r, rocblas_gemm_algo_standard, 0, 0) != rocblas_status_success)
    rc = -11;
  gemm_temp_free(wd, s);
  return rc;
}

}  // namespace qvx
