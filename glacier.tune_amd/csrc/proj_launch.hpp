// proj_launch.hpp -- host-side interface of proj_lora.hip (the projection
// with LoRA adapters) for engine.cpp.
#pragma once

#include <hip/hip_runtime.h>

namespace glacier {

constexpr int kMaxRank = 64;  // LoRA ranks the kernels take (1..64)
constexpr int kMaxProj = 4;   // projections of one input per call

// One projection p of the input: W [out][in] (io dtype), bias [out] fp32 or
// null, A [in][r] and B [r][out] fp32 (A null: no adapter), y [T][out]
// (forward), dy [T][out] (backward), grad_a [in][r] and grad_b [r][out]
// accumulated (+=) when not null.
struct ProjSpec {
  const void* w;
  const float* bias;
  const float* a;
  const float* b;
  float scaling;
  int out;
  void* y;
  const void* dy;
  float* grad_a;
  float* grad_b;
};

struct ProjLaunch {
  int T, in, rank;
  bool io_bf16;
  int n_proj;
  ProjSpec p[kMaxProj];
  const void* x;  // [T][in]
  void* dx;       // [T][in] (backward; overwritten)
  // scratch
  float* yf;    // [T][max out] base product
  float* lr;    // [T][r] X A
  float* dl;    // [n_proj][T][r] dY B^T
  float* dxf;   // [T][in] sum of the base gradients
  float* part;  // [ceil(T/256)][r][max(in, out)] partial gradient sums
};

// The adapter terms of dX for the epilogue (by value, a kernel argument).
struct DxTerms {
  int n;
  const float* dl[kMaxProj];
  const float* a[kMaxProj];
  float scaling[kMaxProj];
};

// Enqueue on st; blas is a rocBLAS handle from create_blas_handle().
hipError_t launch_proj_forward(const ProjLaunch& a, hipStream_t st, void* blas);
hipError_t launch_proj_backward(const ProjLaunch& a, hipStream_t st, void* blas);
void* create_blas_handle();
void destroy_blas_handle(void* h);

}  // namespace glacier
