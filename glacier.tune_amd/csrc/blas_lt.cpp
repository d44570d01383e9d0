// blas_lt.cpp -- hipBLASLt GEMMs for the projection (proj_lora.hip) and the
// LM head (lmhead.hip).
#include "blas_lt.hpp"

#include <hipblaslt/hipblaslt.h>

#include <map>
#include <tuple>

namespace glacier {
namespace {

// One matmul descriptor, four layouts and the heuristic's best zero-workspace algorithm
// per GEMM shape, kept for the handle's life.  No workspace is offered, so no
// algorithm splits the reduction: every result is bitwise repeatable.
struct GemmPlan {
  hipblasLtMatmulDesc_t desc = nullptr;
  hipblasLtMatrixLayout_t a = nullptr, b = nullptr, c = nullptr;
  hipblasLtMatmulAlgo_t algo{};
};

struct Blas {
  hipblasLtHandle_t lt = nullptr;
  std::map<std::tuple<bool, bool, bool, int, int, int, int, int, int>, GemmPlan> plans;

  ~Blas() {
    for (auto& kv : plans) release(kv.second);
    if (lt != nullptr) hipblasLtDestroy(lt);
  }

  // Row-major C [M x N] = alpha op(A) [M x K] op(B) [K x N] + beta C (fp32 C,
  // bf16 or fp32 A and B; leading dimensions are row strides), as the
  // column-major C^T = op(B)^T op(A)^T.
  hipblasStatus_t gemm(bool bf16_in, bool ta, bool tb, int M, int N, int K, float alpha,
                       const void* A, int lda, const void* B, int ldb, float beta, float* C, int ldc,
                       hipStream_t st) {
    const auto key = std::make_tuple(bf16_in, ta, tb, M, N, K, lda, ldb, ldc);
    auto it = plans.find(key);
    if (it == plans.end()) {
      GemmPlan g;
      const hipblasStatus_t e = make_plan(bf16_in, ta, tb, M, N, K, lda, ldb, ldc, g);
      if (e != HIPBLAS_STATUS_SUCCESS) {
        release(g);  // the next call of this shape tries again
        return e;
      }
      it = plans.emplace(key, g).first;
    }
    const GemmPlan& g = it->second;
    return hipblasLtMatmul(lt, g.desc, &alpha, B, g.a, A, g.b, &beta, C, g.c, C, g.c, &g.algo,
                           nullptr, 0, st);
  }

 private:
  static void release(GemmPlan& g) {
    if (g.a != nullptr) hipblasLtMatrixLayoutDestroy(g.a);
    if (g.b != nullptr) hipblasLtMatrixLayoutDestroy(g.b);
    if (g.c != nullptr) hipblasLtMatrixLayoutDestroy(g.c);
    if (g.desc != nullptr) hipblasLtMatmulDescDestroy(g.desc);
    g = GemmPlan{};
  }

  hipblasStatus_t make_plan(bool bf16_in, bool ta, bool tb, int M, int N, int K, int lda, int ldb,
                            int ldc, GemmPlan& g) {
    const hipDataType in_t = bf16_in ? HIP_R_16BF : HIP_R_32F;
    const hipblasOperation_t op_a = tb ? HIPBLAS_OP_T : HIPBLAS_OP_N;  // column-major A' = op(B)^T
    const hipblasOperation_t op_b = ta ? HIPBLAS_OP_T : HIPBLAS_OP_N;  // column-major B' = op(A)^T
    hipblasStatus_t e = hipblasLtMatmulDescCreate(&g.desc, HIPBLAS_COMPUTE_32F, HIP_R_32F);
    if (e == HIPBLAS_STATUS_SUCCESS)
      e = hipblasLtMatmulDescSetAttribute(g.desc, HIPBLASLT_MATMUL_DESC_TRANSA, &op_a, sizeof(op_a));
    if (e == HIPBLAS_STATUS_SUCCESS)
      e = hipblasLtMatmulDescSetAttribute(g.desc, HIPBLASLT_MATMUL_DESC_TRANSB, &op_b, sizeof(op_b));
    const GemmLayouts l = gemm_layouts(ta, tb, M, N, K, lda, ldb, ldc);
    if (e == HIPBLAS_STATUS_SUCCESS)
      e = hipblasLtMatrixLayoutCreate(&g.a, in_t, l.b_first.rows, l.b_first.cols, l.b_first.ld);
    if (e == HIPBLAS_STATUS_SUCCESS)
      e = hipblasLtMatrixLayoutCreate(&g.b, in_t, l.a_second.rows, l.a_second.cols, l.a_second.ld);
    if (e == HIPBLAS_STATUS_SUCCESS)
      e = hipblasLtMatrixLayoutCreate(&g.c, HIP_R_32F, l.c.rows, l.c.cols, l.c.ld);
    hipblasLtMatmulPreference_t pref = nullptr;
    if (e == HIPBLAS_STATUS_SUCCESS) e = hipblasLtMatmulPreferenceCreate(&pref);
    const uint64_t no_workspace = 0;
    if (e == HIPBLAS_STATUS_SUCCESS)
      e = hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES,
                                                &no_workspace, sizeof(no_workspace));
    // The GEMMs run with no workspace: take the heuristic's best algorithm
    // that needs none, and fail the plan (an error status, no GEMM) if none
    // of those returned does.
    constexpr int kCand = 8;
    hipblasLtMatmulHeuristicResult_t res[kCand];
    int found = 0;
    if (e == HIPBLAS_STATUS_SUCCESS)
      e = hipblasLtMatmulAlgoGetHeuristic(lt, g.desc, g.a, g.b, g.c, g.c, pref, kCand, res, &found);
    if (pref != nullptr) hipblasLtMatmulPreferenceDestroy(pref);
    int pick = -1;
    for (int i = 0; e == HIPBLAS_STATUS_SUCCESS && i < found && pick < 0; ++i)
      if (res[i].state == HIPBLAS_STATUS_SUCCESS && res[i].workspaceSize == 0) pick = i;
    if (e == HIPBLAS_STATUS_SUCCESS && pick < 0) e = HIPBLAS_STATUS_NOT_SUPPORTED;
    if (e == HIPBLAS_STATUS_SUCCESS) g.algo = res[pick].algo;
    return e;
  }
};

}  // namespace

// Stored shapes (rows x cols, column-major): the caller's B as N x K (tb) or
// K x N, its A as K x M or M x K (ta), C as N x M; leading dimensions are the
// caller's row strides.
GemmLayouts gemm_layouts(bool ta, bool tb, int M, int N, int K, int lda, int ldb, int ldc) {
  GemmLayouts l;
  l.b_first = GemmOperand{tb ? K : N, tb ? N : K, ldb};
  l.a_second = GemmOperand{ta ? M : K, ta ? K : M, lda};
  l.c = GemmOperand{N, M, ldc};
  return l;
}

void* create_blas_handle() {
  Blas* b = new Blas;
  if (hipblasLtCreate(&b->lt) != HIPBLAS_STATUS_SUCCESS) {
    b->lt = nullptr;
    delete b;
    return nullptr;
  }
  return b;
}

void destroy_blas_handle(void* h) { delete static_cast<Blas*>(h); }

hipError_t blas_gemm(void* h, bool bf16_in, bool ta, bool tb, int M, int N, int K, float alpha,
                     const void* A, int lda, const void* B, int ldb, float beta, float* C, int ldc,
                     hipStream_t st) {
  const hipblasStatus_t e = static_cast<Blas*>(h)->gemm(bf16_in, ta, tb, M, N, K, alpha, A, lda, B,
                                                         ldb, beta, C, ldc, st);
  return e == HIPBLAS_STATUS_SUCCESS ? hipSuccess : hipErrorLaunchFailure;
}

}  // namespace glacier
