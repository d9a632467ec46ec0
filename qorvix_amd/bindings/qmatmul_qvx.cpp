// qmatmul_qvx.cpp -- the reference runtime's operator and dequantisation entry points served by the
// MI355X engine (libqvx.so): a drop-in replacement for runtime/src/qmatmul.cpp and the dequant
// functions of runtime/src/dequant.cpp, defining the functions its headers declare
// (runtime/include/qorvix/runtime/qmatmul.hpp:14-36, dequant.hpp:12-21) on the C ABI of
// include/qvx.h.  Host pointers, synchronous -- the reference's CPU calling convention.  Every
// `false` case of the reference is a non-QVX_OK status before any work.  Build it into the
// reference's runtime library in place of those two files and link -lqvx.
#include "qorvix/runtime/dequant.hpp"
#include "qorvix/runtime/qmatmul.hpp"
#include "qvx.h"

namespace qorvix::runtime {

bool qmatmulSupports(std::uint32_t ggmlType) { return qvx_supports(ggmlType) != 0; }

bool qmatmul(float* out, const void* weight, std::uint32_t ggmlType, const float* x, int rows, int cols) {
  return qvx_qmatmul_host(out, weight, ggmlType, x, rows, cols) == QVX_OK;
}

bool qmatmulN(float* out, const void* weight, std::uint32_t ggmlType, const float* X, int nVec, int rows,
              int cols) {
  return qvx_qmatmul_n_host(out, weight, ggmlType, X, nVec, rows, cols) == QVX_OK;
}

bool dequantRow(const void* weight, std::uint32_t ggmlType, int cols, int row, float* dst) {
  return qvx_dequant_row_host(weight, ggmlType, cols, row, dst) == QVX_OK;
}

float fp16ToFloat(std::uint16_t h) { return qvx_fp16_to_float(h); }

float bf16ToFloat(std::uint16_t b) { return qvx_bf16_to_float(b); }

bool canDequantize(std::uint32_t ggmlType) { return qvx_can_dequantize(ggmlType) != 0; }

bool dequantize(std::uint32_t ggmlType, const void* src, float* dst, std::size_t nElements) {
  return qvx_dequantize_host(ggmlType, src, dst, nElements) == QVX_OK;
}

}  // namespace qorvix::runtime
