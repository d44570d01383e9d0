// blas_lt.hpp -- the library's hipBLASLt GEMMs (blas_lt.cpp): one handle per
// engine, with a plan (descriptor, layouts, algorithm) cached per shape.
#pragma once

#include <hip/hip_runtime.h>

namespace glacier {

// A hipBLASLt handle with its plan cache, or null on failure.
void* create_blas_handle();
void destroy_blas_handle(void* h);

// Row-major C [M x N] = alpha op(A) [M x K] op(B) [K x N] + beta C on st:
// fp32 C and accumulation, A and B bf16 (bf16_in) or fp32; leading
// dimensions are row strides.  Without workspace (no split reductions), so
// every result is bitwise repeatable.  hipErrorLaunchFailure if hipBLASLt
// has no algorithm or fails.
hipError_t blas_gemm(void* h, bool bf16_in, bool ta, bool tb, int M, int N, int K, float alpha,
                     const void* A, int lda, const void* B, int ldb, float beta, float* C, int ldc,
                     hipStream_t st);

}  // namespace glacier
