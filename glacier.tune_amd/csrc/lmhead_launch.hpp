// lmhead_launch.hpp -- host-side interface of lmhead.hip (the LM-head
// cross-entropy loss and its hidden-state gradient) for engine.cpp.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <string>
#include <vector>

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

// ---- shared by the kernels, engine.cpp and host-side bounds checks -------

// The kept rows of a call (the reference's filter, FusedCrossEntropyLoss.cs:53,
// :190): rows[] and tgts[] per kept row, src_of[t] its packed index or -1.
void lmhead_rows(const int32_t* targets, int T, int V, std::vector<int>& rows,
                 std::vector<int>& tgts, std::vector<int>& src_of);

// Sets a.n_valid, a.ldl (V rounded up to 8) and a.chunk (kept rows per pass,
// logits plus bf16 dlogits within kLmHeadChunkBytes).
void lmhead_shape(LmHeadLaunch& a, int n_valid);

// Device scratch (bytes) that a launch shaped by lmhead_shape reads and writes.
struct LmHeadScratch {
  size_t idx;       // rows, targets, src_of: int32
  size_t hv;        // packed hidden rows (io dtype)
  size_t logits;    // fp32
  size_t dl;        // bf16 dlogits (0 in the fp32 mode: the logits buffer)
  size_t dhv;       // packed fp32 gradient (0 without a gradient)
  size_t row_loss;  // n_valid row terms and the loss
};
LmHeadScratch lmhead_scratch(const LmHeadLaunch& a);

// Index arithmetic of the kernels, for the device and the host check.
struct CeGatherAt {
  int i, p;  // packed row, 16-byte piece
};
__host__ __device__ inline int ce_gather_pieces(int H, int esz) { return H * esz / 16; }
__host__ __device__ inline CeGatherAt ce_gather_at(long idx, int per_row) {
  return CeGatherAt{static_cast<int>(idx / per_row), static_cast<int>(idx % per_row)};
}
struct CeScatterAt {
  int t, c;  // row, first of its four columns
};
__host__ __device__ inline CeScatterAt ce_scatter_at(long idx, int q4) {
  return CeScatterAt{static_cast<int>(idx / q4), 4 * static_cast<int>(idx % q4)};
}
constexpr int kCeThreads = 256;

// Walks every access launch_lmhead's kernels and GEMMs make for `a` (whose
// index arrays are given as host copies), with the grids launch_lmhead uses,
// and checks it against the scratch sizes `s` and the caller's tensors
// (elements).  Returns "" when every access is in bounds, else the first one
// that is not.  Host only: no device work.
std::string lmhead_check_bounds(const LmHeadLaunch& a, const LmHeadScratch& s, const int* rows,
                                const int* targets, const int* src_of, size_t hidden_elems,
                                size_t weight_elems, size_t d_hidden_elems);

}  // namespace glacier
