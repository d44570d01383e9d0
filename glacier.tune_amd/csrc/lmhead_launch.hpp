// lmhead_launch.hpp -- host-side interface of lmhead.hip (the LM-head
// cross-entropy loss and its hidden-state gradient) for engine.cpp.
#pragma once

#include <hip/hip_runtime.h>

namespace glacier {

// Logits (fp32) plus dlogits held at once per chunk of kept rows.
constexpr long kLmHeadChunkBytes = 2L << 30;

struct LmHeadLaunch {
  int T, H, V;    // rows of hidden, hidden size, vocabulary
  int n_valid;    // rows whose target is in [0, V)
  int ldl;        // row stride of the logits: V rounded up to 8
  int chunk;      // kept rows per pass through the two GEMMs
  bool io_bf16;   // hidden, weight, d_hidden bf16 (bf16 GEMM operands)
  const void* hidden;  // [T][H]
  const void* weight;  // [V][H]
  void* d_hidden;      // [T][H], or null: loss only
  // device scratch
  const int* rows;     // [n_valid] index of each kept row
  const int* targets;  // [n_valid] its target
  const int* src_of;   // [T] packed index of each row, or -1
  void* hv;            // [chunk][H] packed hidden rows (io dtype)
  float* logits;       // [chunk][ldl]
  void* dl;            // [chunk][ldl] dlogits: bf16, or the logits buffer itself (fp32)
  float* dhv;          // [n_valid][H] packed gradient
  float* row_loss;     // [n_valid] lse - target logit
  float* loss;         // [1] the mean
};

// Enqueue on st (blas: create_blas_handle()); the caller copies a.loss back.
hipError_t launch_lmhead(const LmHeadLaunch& a, hipStream_t st, void* blas);

}  // namespace glacier
