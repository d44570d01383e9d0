// proj_lora.hip -- the projection step either side of attention, on the
// device: a frozen base projection plus a trainable LoRA adapter, for the q,
// k and v projections of one normalised input (GpuLoraEngine.ForwardQKV,
// GpuLoraEngine.Forward.cs:205-245, whose LoRA delta the reference adds on
// the host, AddLoraDeltaHost :366-399), and the reverse
// (LoraAdapter.Backward, LoraAdapter.cs:190-247).
//
// Per projection p, with X [T][in], W_p [out][in], A_p [in][r], B_p [r][out]:
//   forward   Y_p  = X W_p^T + bias_p + s_p (X A_p) B_p
//   backward  dX   = sum_p dY_p W_p + s_p (dY_p B_p^T) A_p^T
//             dA_p += s_p X^T (dY_p B_p^T),  dB_p += s_p (X A_p)^T dY_p
// The base products (the only large ones) are rocBLAS GEMMs with fp32
// results in scratch; everything of rank r is done here, fused into the
// epilogues that add the deltas and write the caller's dtype:
//   lora_down      L = X A             one wave per row, lanes over in
//   proj_epilogue  Y = io(Yf + bias + s L B)
//   lora_dl        dL = dY B^T         one wave per row, lanes over out
//   lora_grad      partial column sums of X^T dL or L^T dY over token blocks
//   lora_grad_sum  grad += s * (sum of the partials in block order)
//   dx_epilogue    dX = io(dXf + sum_p s_p dL_p A_p^T)
// Every sum has a fixed order (rocBLAS runs with atomics disallowed), so
// results are bitwise repeatable.
#include "attn_common.hpp"
#include "proj_launch.hpp"

#include <rocblas/rocblas.h>

namespace glacier {
namespace {

constexpr int kProjThreads = 256;
constexpr int kGradRows = 256;  // tokens per partial sum of the adapter gradients

template <typename IO>
__device__ inline float ld(const IO* p) {
  return to_f32(*p);
}

// Sum over the 64 lanes of a wave in a fixed order (every lane gets it).
__device__ inline float wave_sum(float x) {
  x = lanes_sum<32>(x);
  return x + __shfl_xor(x, 32);
}

// L[t][j] = sum_k X[t][k] A[k][j]; grid.x = rows / 4, 4 waves per block.
// Lane l takes k = l, l + 64, ... in ascending order.
template <typename IO>
__global__ __launch_bounds__(kProjThreads) void lora_down_kernel(const IO* __restrict__ x,
                                                                 const float* __restrict__ a,
                                                                 float* __restrict__ lr, int T,
                                                                 int in, int rank) {
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (t >= T) return;
  float acc[kMaxRank];
#pragma unroll
  for (int j = 0; j < kMaxRank; ++j) acc[j] = 0.0f;
  const IO* row = x + (long)t * in;
  for (int k = lane; k < in; k += 64) {
    const float xv = ld(row + k);
    const float* ar = a + (long)k * rank;
#pragma unroll
    for (int j = 0; j < kMaxRank; ++j)
      if (j < rank) acc[j] += xv * ar[j];
  }
#pragma unroll
  for (int j = 0; j < kMaxRank; ++j) {
    if (j < rank) {
      const float v = wave_sum(acc[j]);
      if (lane == 0) lr[(long)t * rank + j] = v;
    }
  }
}

// dL[t][j] = sum_n dY[t][n] B[j][n]; lane l takes n = l, l + 64, ...
template <typename IO>
__global__ __launch_bounds__(kProjThreads) void lora_dl_kernel(const IO* __restrict__ dy,
                                                               const float* __restrict__ b,
                                                               float* __restrict__ dl, int T,
                                                               int out, int rank) {
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (t >= T) return;
  float acc[kMaxRank];
#pragma unroll
  for (int j = 0; j < kMaxRank; ++j) acc[j] = 0.0f;
  const IO* row = dy + (long)t * out;
  for (int n = lane; n < out; n += 64) {
    const float g = ld(row + n);
#pragma unroll
    for (int j = 0; j < kMaxRank; ++j)
      if (j < rank) acc[j] += g * b[(long)j * out + n];
  }
#pragma unroll
  for (int j = 0; j < kMaxRank; ++j) {
    if (j < rank) {
      const float v = wave_sum(acc[j]);
      if (lane == 0) dl[(long)t * rank + j] = v;
    }
  }
}

// Y[t][n] = io(Yf[t][n] + bias[n] + sum_j (s L[t][j]) B[j][n]), 4 columns
// per thread (out % 4 == 0), the terms added in the reference's order
// (LoraAdapter.cs:141-150, LoraKernels.cs:103-112).
template <typename IO>
__global__ __launch_bounds__(kProjThreads) void proj_epilogue_kernel(
    const float* __restrict__ yf, const float* __restrict__ bias, const float* __restrict__ lr,
    const float* __restrict__ b, float scaling, IO* __restrict__ y, int T, int out, int rank) {
  const long idx = (long)blockIdx.x * kProjThreads + threadIdx.x;
  const int q4 = out / 4;
  if (idx >= (long)T * q4) return;
  const int t = (int)(idx / q4), n = 4 * (int)(idx % q4);
  f32x4 v = *reinterpret_cast<const f32x4*>(yf + (long)t * out + n);
  if (bias != nullptr) {
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] += bias[n + e];
  }
  if (lr != nullptr) {
    for (int j = 0; j < rank; ++j) {
      const float s = lr[(long)t * rank + j] * scaling;
      const f32x4 bj = *reinterpret_cast<const f32x4*>(b + (long)j * out + n);
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] += s * bj[e];
    }
  }
  store4(y + (long)t * out + n, v);
}

// Partial sums P[c][j][col] = sum_{t in block c} U[t][col] V[t][j] over a
// block of kGradRows tokens (ascending), for the adapter gradients:
// grad_a: U = X [T][in],  V = dL [T][r];  grad_b: U = dY [T][out], V = L [T][r].
// grid (ceil(cols / 256), blocks of tokens); one column per thread.
template <typename IO>
__global__ __launch_bounds__(kProjThreads) void lora_grad_kernel(const IO* __restrict__ u,
                                                                 const float* __restrict__ v,
                                                                 float* __restrict__ part, int T,
                                                                 int cols, int rank) {
  const int col = blockIdx.x * kProjThreads + threadIdx.x;
  const int t0 = blockIdx.y * kGradRows, t1 = min(T, t0 + kGradRows);
  if (col >= cols) return;
  float acc[kMaxRank];
#pragma unroll
  for (int j = 0; j < kMaxRank; ++j) acc[j] = 0.0f;
  for (int t = t0; t < t1; ++t) {
    const float uv = ld(u + (long)t * cols + col);
    const float* vr = v + (long)t * rank;
#pragma unroll
    for (int j = 0; j < kMaxRank; ++j)
      if (j < rank) acc[j] += uv * vr[j];
  }
  float* pr = part + (long)blockIdx.y * rank * cols;
#pragma unroll
  for (int j = 0; j < kMaxRank; ++j)
    if (j < rank) pr[(long)j * cols + col] = acc[j];
}

// grad[col][j] (transposed: grad_a is [in][r]) or grad[j][col] (grad_b is
// [r][out]) += s * sum_c P[c][j][col], blocks in ascending order.
__global__ __launch_bounds__(kProjThreads) void lora_grad_sum_kernel(
    const float* __restrict__ part, int nblk, int cols, int rank, float scaling,
    float* __restrict__ grad, int transposed) {
  const long idx = (long)blockIdx.x * kProjThreads + threadIdx.x;
  if (idx >= (long)cols * rank) return;
  const int j = (int)(idx / cols), col = (int)(idx % cols);
  float sum = 0.0f;
  for (int c = 0; c < nblk; ++c) sum += part[((long)c * rank + j) * cols + col];
  float* g = transposed ? grad + (long)col * rank + j : grad + (long)j * cols + col;
  *g += sum * scaling;
}

// dX[t][k] = io(dXf[t][k] + sum_p s_p sum_j dL_p[t][j] A_p[k][j]), 4
// columns per thread (in % 4 == 0), projections in order.
template <typename IO>
__global__ __launch_bounds__(kProjThreads) void dx_epilogue_kernel(const float* __restrict__ dxf,
                                                                   DxTerms terms,
                                                                   IO* __restrict__ dx, int T,
                                                                   int in, int rank) {
  const long idx = (long)blockIdx.x * kProjThreads + threadIdx.x;
  const int q4 = in / 4;
  if (idx >= (long)T * q4) return;
  const int t = (int)(idx / q4), k = 4 * (int)(idx % q4);
  f32x4 v = *reinterpret_cast<const f32x4*>(dxf + (long)t * in + k);
  for (int p = 0; p < terms.n; ++p) {
    const float* dl = terms.dl[p] + (long)t * rank;
    const float* a = terms.a[p];
    f32x4 dot = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int j = 0; j < rank; ++j) {
      const float d = dl[j];
#pragma unroll
      for (int e = 0; e < 4; ++e) dot[e] += d * a[(long)(k + e) * rank + j];
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] += dot[e] * terms.scaling[p];
  }
  store4(dx + (long)t * in + k, v);
}

unsigned blocks(long n, int per) { return static_cast<unsigned>((n + per - 1) / per); }

rocblas_status gemm(rocblas_handle h, bool bf16, rocblas_operation ta, rocblas_operation tb, int m,
                    int n, int k, const void* a, int lda, const void* b, int ldb, float beta,
                    float* c, int ldc) {
  const float alpha = 1.0f;
  const rocblas_datatype in_t = bf16 ? rocblas_datatype_bf16_r : rocblas_datatype_f32_r;
  return rocblas_gemm_ex(h, ta, tb, m, n, k, &alpha, a, in_t, lda, b, in_t, ldb, &beta, c,
                         rocblas_datatype_f32_r, ldc, c, rocblas_datatype_f32_r, ldc,
                         rocblas_datatype_f32_r, rocblas_gemm_algo_standard, 0,
                         rocblas_gemm_flags_none);
}

#define PROJ_CHECK_BLAS(expr)                                   \
  do {                                                          \
    if ((expr) != rocblas_status_success) return hipErrorLaunchFailure; \
  } while (0)

template <typename IO>
hipError_t forward_impl(const ProjLaunch& a, hipStream_t st, rocblas_handle h) {
  constexpr bool BF = sizeof(IO) == 2;
  const IO* x = static_cast<const IO*>(a.x);
  for (int p = 0; p < a.n_proj; ++p) {
    const ProjSpec& s = a.p[p];
    // Yf = X W^T: column-major Yf^T [out x T] = W (W^T stored) x X^T
    PROJ_CHECK_BLAS(gemm(h, BF, rocblas_operation_transpose, rocblas_operation_none, s.out, a.T,
                         a.in, s.w, a.in, a.x, a.in, 0.0f, a.yf, s.out));
    const bool lora = s.a != nullptr;
    if (lora) {
      hipLaunchKernelGGL(lora_down_kernel<IO>, dim3(blocks(a.T, 4)), dim3(kProjThreads), 0, st, x,
                         s.a, a.lr, a.T, a.in, a.rank);
      GL_CHECK(hipGetLastError());
    }
    hipLaunchKernelGGL(proj_epilogue_kernel<IO>, dim3(blocks((long)a.T * (s.out / 4), kProjThreads)),
                       dim3(kProjThreads), 0, st, a.yf, s.bias, lora ? a.lr : nullptr, s.b,
                       s.scaling, static_cast<IO*>(s.y), a.T, s.out, a.rank);
    GL_CHECK(hipGetLastError());
  }
  return hipSuccess;
}

template <typename IO>
hipError_t backward_impl(const ProjLaunch& a, hipStream_t st, rocblas_handle h) {
  constexpr bool BF = sizeof(IO) == 2;
  const IO* x = static_cast<const IO*>(a.x);
  const int nblk = (a.T + kGradRows - 1) / kGradRows;
  DxTerms terms{};
  for (int p = 0; p < a.n_proj; ++p) {
    const ProjSpec& s = a.p[p];
    // dXf (+)= dY W: column-major dXf^T [in x T] = W^T (W stored) x dY^T
    PROJ_CHECK_BLAS(gemm(h, BF, rocblas_operation_none, rocblas_operation_none, a.in, a.T, s.out,
                         s.w, a.in, s.dy, s.out, p == 0 ? 0.0f : 1.0f, a.dxf, a.in));
    if (s.a == nullptr) continue;
    const IO* dy = static_cast<const IO*>(s.dy);
    float* dl = a.dl + (long)p * a.T * a.rank;
    hipLaunchKernelGGL(lora_dl_kernel<IO>, dim3(blocks(a.T, 4)), dim3(kProjThreads), 0, st, dy, s.b,
                       dl, a.T, s.out, a.rank);
    GL_CHECK(hipGetLastError());
    if (s.grad_b != nullptr) {
      hipLaunchKernelGGL(lora_down_kernel<IO>, dim3(blocks(a.T, 4)), dim3(kProjThreads), 0, st, x,
                         s.a, a.lr, a.T, a.in, a.rank);
      GL_CHECK(hipGetLastError());
      hipLaunchKernelGGL(lora_grad_kernel<IO>, dim3(blocks(s.out, kProjThreads), nblk),
                         dim3(kProjThreads), 0, st, dy, a.lr, a.part, a.T, s.out, a.rank);
      GL_CHECK(hipGetLastError());
      hipLaunchKernelGGL(lora_grad_sum_kernel, dim3(blocks((long)s.out * a.rank, kProjThreads)),
                         dim3(kProjThreads), 0, st, a.part, nblk, s.out, a.rank, s.scaling,
                         s.grad_b, 0);
      GL_CHECK(hipGetLastError());
    }
    if (s.grad_a != nullptr) {
      hipLaunchKernelGGL(lora_grad_kernel<IO>, dim3(blocks(a.in, kProjThreads), nblk),
                         dim3(kProjThreads), 0, st, x, dl, a.part, a.T, a.in, a.rank);
      GL_CHECK(hipGetLastError());
      hipLaunchKernelGGL(lora_grad_sum_kernel, dim3(blocks((long)a.in * a.rank, kProjThreads)),
                         dim3(kProjThreads), 0, st, a.part, nblk, a.in, a.rank, s.scaling,
                         s.grad_a, 1);
      GL_CHECK(hipGetLastError());
    }
    terms.dl[terms.n] = dl;
    terms.a[terms.n] = s.a;
    terms.scaling[terms.n] = s.scaling;
    ++terms.n;
  }
  hipLaunchKernelGGL(dx_epilogue_kernel<IO>, dim3(blocks((long)a.T * (a.in / 4), kProjThreads)),
                     dim3(kProjThreads), 0, st, a.dxf, terms, static_cast<IO*>(a.dx), a.T, a.in,
                     a.rank);
  GL_CHECK(hipGetLastError());
  return hipSuccess;
}

}  // namespace

hipError_t launch_proj_forward(const ProjLaunch& a, hipStream_t st, void* blas) {
  auto h = static_cast<rocblas_handle>(blas);
  if (rocblas_set_stream(h, st) != rocblas_status_success) return hipErrorInvalidHandle;
  return a.io_bf16 ? forward_impl<bf16>(a, st, h) : forward_impl<float>(a, st, h);
}

hipError_t launch_proj_backward(const ProjLaunch& a, hipStream_t st, void* blas) {
  auto h = static_cast<rocblas_handle>(blas);
  if (rocblas_set_stream(h, st) != rocblas_status_success) return hipErrorInvalidHandle;
  return a.io_bf16 ? backward_impl<bf16>(a, st, h) : backward_impl<float>(a, st, h);
}

// rocBLAS handle owned by an engine; atomics are disallowed so that every
// GEMM is bitwise repeatable.
void* create_blas_handle() {
  rocblas_handle h = nullptr;
  if (rocblas_create_handle(&h) != rocblas_status_success) return nullptr;
  if (rocblas_set_atomics_mode(h, rocblas_atomics_not_allowed) != rocblas_status_success) {
    rocblas_destroy_handle(h);
    return nullptr;
  }
  return h;
}

void destroy_blas_handle(void* h) {
  if (h != nullptr) rocblas_destroy_handle(static_cast<rocblas_handle>(h));
}

}  // namespace glacier
