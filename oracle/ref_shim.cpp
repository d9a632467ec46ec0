// ref_shim.cpp -- C entry points onto the reference's own CPU operator, for ctypes.
//
// TEST INFRASTRUCTURE ONLY (see qvx_oracle.c).  Linked with the reference's unmodified sources
// runtime/src/{dequant,qmatmul,cpu_features,ops}.cpp and gguf/src/gguf_types.cpp, compiled where they
// lie under /root/reference by oracle/Makefile into oracle/_ref/.  Nothing here restates the
// reference; each function forwards to the declaration cited beside it.
#include <cstddef>
#include <cstdint>

#include "qorvix/runtime/cpu_features.hpp"  // runtime/include/qorvix/runtime/cpu_features.hpp:38-45
#include "qorvix/runtime/dequant.hpp"       // runtime/include/qorvix/runtime/dequant.hpp:12-21
#include "qorvix/runtime/ops.hpp"           // runtime/include/qorvix/runtime/ops.hpp:11,35-38
#include "qorvix/runtime/qmatmul.hpp"       // runtime/include/qorvix/runtime/qmatmul.hpp:14-36

namespace rt = qorvix::runtime;

extern "C" {
__attribute__((visibility("default"))) int qvxr_supports(std::uint32_t t) { return rt::qmatmulSupports(t); }
__attribute__((visibility("default"))) int qvxr_can_dequantize(std::uint32_t t) { return rt::canDequantize(t); }
__attribute__((visibility("default"))) float qvxr_fp16_to_float(std::uint16_t h) { return rt::fp16ToFloat(h); }
__attribute__((visibility("default"))) int qvxr_dequantize(std::uint32_t t, const void* src, float* dst,
                                                           std::size_t n) {
  return rt::dequantize(t, src, dst, n);
}
__attribute__((visibility("default"))) int qvxr_qmatmul(float* out, const void* w, std::uint32_t t,
                                                        const float* x, int rows, int cols) {
  return rt::qmatmul(out, w, t, x, rows, cols);
}
__attribute__((visibility("default"))) int qvxr_qmatmul_n(float* out, const void* w, std::uint32_t t,
                                                          const float* X, int nvec, int rows, int cols) {
  return rt::qmatmulN(out, w, t, X, nvec, rows, cols);
}
__attribute__((visibility("default"))) int qvxr_dequant_row(const void* w, std::uint32_t t, int cols, int row,
                                                            float* dst) {
  return rt::dequantRow(w, t, cols, row, dst);
}
__attribute__((visibility("default"))) const char* qvxr_dot_kernel() { return rt::cpu::activeDotKernel(); }
__attribute__((visibility("default"))) void qvxr_rmsnorm(float* out, const float* x, const float* w, int n,
                                                         float eps) {
  rt::ops::rmsnorm(out, x, w, n, eps);
}
__attribute__((visibility("default"))) void qvxr_swiglu(float* out, const float* gate, const float* up, int n) {
  rt::ops::swiglu(out, gate, up, n);
}
}
