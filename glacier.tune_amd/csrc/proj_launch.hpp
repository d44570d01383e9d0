// proj_launch.hpp -- host-side interface of proj_lora.hip (the projection
// with LoRA adapters) for engine.cpp.
#pragma once

#include <hip/hip_runtime.h>

namespace glacier {

constexpr int kMaxRank = 64;  // largest LoRA rank taken
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
  // scratch (fp32), sized by proj_scratch_need
  float* yf;       // forward: [T][out_p] base products, one after another
  float* dxf;      // backward: [T][in] sum_p dY_p W_p
  float* lowrank;  // [slot][T][r] X A_p and dY_p B_p^T
  float* part;     // split sums of those products
};

// Floats of each ProjLaunch scratch buffer for a forward or backward call.
struct ProjScratchNeed {
  long yf, dxf, lowrank, part;
};
ProjScratchNeed proj_scratch_need(const ProjLaunch& a, bool backward);

// Enqueue on st; blas is a handle from create_blas_handle() (blas_lt.hpp).
hipError_t launch_proj_forward(const ProjLaunch& a, hipStream_t st, void* blas);
hipError_t launch_proj_backward(const ProjLaunch& a, hipStream_t st, void* blas);

}  // namespace glacier
