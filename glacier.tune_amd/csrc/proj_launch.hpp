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
                   // ([nsplit][T][out_p] for a narrow projection of bf16 tensors)
  float* dxf;      // backward: [T][in] sum_p dY_p W_p over the library-GEMM
                   // projections, then [T][in] over the narrow ones
  float* lowrank;  // [slot][T][r] X A_p and dY_p B_p^T
  float* part;     // split sums of those products
};

// ---- the narrow base products on the library's own GEMM (proj_gemm.hip) ----
// bf16 tensors, inputs a multiple of 64 and at most kNarrowMaxOut outputs,
// also a multiple of 64 (the k and v projections of a GQA block).
constexpr int kNarrowMaxOut = 1024;

struct NarrowJob {
  const void* w;   // W_p [n][in] (bf16)
  const void* dy;  // backward: dY_p [T][n] (bf16)
  float* c;        // forward: fp32 partials [nsplit][T][n]
  int n;           // outputs of the projection
  int first;       // forward: its first workgroup (set by launch_narrow_fwd)
};

// Yf_p[s] = X W_p^T over input slice s (kchunk inputs) for each job.
struct NarrowFwd {
  const void* x;  // [T][K] (bf16)
  int T, K, nsplit, kchunk, n;
  NarrowJob j[kMaxProj];
};

// dXf2 [T][K] = sum over the jobs of dY_p W_p (K = the input features).
struct NarrowBwd {
  int T, K;
  float* c;
  int n;
  NarrowJob j[kMaxProj];
};

bool narrow_gemm_fits(int in_features, int out_features);
// Input slices of a forward launch: 1, 2 or 4, so that the launch has about
// a workgroup per CU when the tiles alone are fewer.
int narrow_fwd_splits(int T, int total_feature_tiles);
int narrow_feature_tiles(int out_features);
hipError_t launch_narrow_fwd(NarrowFwd a, hipStream_t st);
hipError_t launch_narrow_bwd(const NarrowBwd& a, hipStream_t st);

// ---- the wide base products on the library's own GEMM (proj_gemm.hip) ----
// bf16 tensors, inputs and outputs multiples of 128 (the q projection).
struct WideJob {
  const void* w;   // W_z [n][K] (bf16)
  const void* dy;  // dY_z [T][n] (bf16)
  int n;           // outputs of the projection
};
// c [T][n] = X W^T (fp32), one projection.
struct WideFwd {
  const void* x;  // [T][K] (bf16)
  const void* w;  // [n][K] (bf16)
  float* c;
  int T, K, n;
};
// c [T][K] = sum over the jobs of dY_z W_z (fp32); accumulate (generic
// kernel only): c += instead.
struct WideBwd {
  float* c;
  int T, K, n;
  WideJob j[kMaxProj];
  bool accumulate;
};
bool wide_gemm_fits(int in_features, int out_features);
hipError_t launch_wide_fwd(const WideFwd& a, hipStream_t st);
hipError_t launch_wide_bwd(const WideBwd& a, hipStream_t st);

// ---- every other projection: the same two products on fp32 MFMAs, any ----
// shape, fp32 or bf16 operands (io_bf16) converted to fp32 on load
hipError_t launch_generic_fwd(const WideFwd& a, bool io_bf16, hipStream_t st);
hipError_t launch_generic_bwd(const WideBwd& a, bool io_bf16, hipStream_t st);

// Floats of each ProjLaunch scratch buffer for a forward or backward call.
struct ProjScratchNeed {
  long yf, dxf, lowrank, part;
};
ProjScratchNeed proj_scratch_need(const ProjLaunch& a, bool backward);

// Enqueue on st.
hipError_t launch_proj_forward(const ProjLaunch& a, hipStream_t st);
hipError_t launch_proj_backward(const ProjLaunch& a, hipStream_t st);

}  // namespace glacier
