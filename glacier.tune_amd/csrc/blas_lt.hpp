// blas_lt.hpp -- the library's hipBLASLt GEMMs (blas_lt.cpp): one handle per
// engine, with a plan (descriptor, layouts, algorithm) cached per shape.
#pragma once

#include <hip/hip_runtime.h>

namespace glacier {

// A hipBLASLt handle with its plan cache, or null on failure.
void* create_blas_handle();
void destroy_blas_handle(void* h);

// The stored extent of one hipBLASLt operand: a column-major matrix of
// `rows` x `cols` elements with leading dimension `ld` (elements), so it
// touches elements [0, ld * (cols - 1) + rows) from its base.
struct GemmOperand {
  int rows, cols, ld;
  long long elements() const { return rows <= 0 || cols <= 0 ? 0 : (long long)ld * (cols - 1) + rows; }
};

// The three layouts blas_gemm describes to hipBLASLt for one GEMM (the
// first operand it is given is the caller's B, the second the caller's A;
// see blas_gemm), so that host code can check their extents against the
// buffers before anything runs.
struct GemmLayouts {
  GemmOperand b_first, a_second, c;
};
GemmLayouts gemm_layouts(bool ta, bool tb, int M, int N, int K, int lda, int ldb, int ldc);

// Row-major C [M x N] = alpha op(A) [M x K] op(B) [K x N] + beta C on st:
// fp32 C and accumulation, A and B bf16 (bf16_in) or fp32; leading
// dimensions are row strides.  Without workspace (no split reductions), so
// every result is bitwise repeatable.  hipErrorLaunchFailure if hipBLASLt
// has no algorithm or fails.
hipError_t blas_gemm(void* h, bool bf16_in, bool ta, bool tb, int M, int N, int K, float alpha,
                     const void* A, int lda, const void* B, int ldb, float beta, float* C, int ldc,
                     hipStream_t st);

}  // namespace glacier
