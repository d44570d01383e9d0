// norm_launch.hpp -- host-side interface of rmsnorm.hip (the residual add and
// RMSNorm) for engine.cpp.
#pragma once

#include <hip/hip_runtime.h>

#include "attn_launch.hpp"  // KernelTimer

namespace glacier {

constexpr int kNormMaxN = 8192;  // widest row taken (32 chunks of 4 per lane)

// Forward: x1 = x + delta (delta null: x1 = x, not written), y = RMSNorm(x1) w.
// Activations [rows][n] in the io dtype, w [n] fp32.
struct NormFwd {
  int rows, n;
  float eps;
  bool io_bf16;
  const void* x;
  const void* delta;  // or null
  const float* w;
  void* x1;  // written when delta is given
  void* y;
};

// Backward: dx = RMSNormBackward(dy; x, w) + d_residual (null: nothing added);
// d_weight += sum over rows of dy x r when not null (rstd: [rows] scratch then;
// dy_w: the dy that sum reads, a copy of dy when dx overwrites it).
struct NormBwd {
  int rows, n;
  float eps;
  bool io_bf16;
  const void* dy;
  const void* x;
  const float* w;
  const void* d_residual;
  void* dx;
  float* d_weight;
  float* rstd;
  const void* dy_w;
};

// Enqueue on st; tm (may be null) times the launches when enabled.
hipError_t launch_rmsnorm_forward(const NormFwd& a, hipStream_t st, KernelTimer* tm);
hipError_t launch_rmsnorm_backward(const NormBwd& a, hipStream_t st, KernelTimer* tm);

}  // namespace glacier
