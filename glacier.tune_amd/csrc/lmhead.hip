// lmhead.hip -- the LM-head cross-entropy loss over the vocabulary and its
// gradient with respect to the final hidden states, on the device
// (FusedCrossEntropyLoss.ComputeLoss / ComputeLossAndGradients,
// src/Glacier.Tune/Kernels/FusedCrossEntropyLoss.cs:38-364):
//   loss  = mean over rows with a target in [0, V) of lse(h W^T) - (h W^T)[target]
//   dh    = (softmax(h W^T) - onehot(target)) W / n,  zero for dropped rows.
// The reference streams 4096-wide vocabulary tiles through host or device
// memory so as never to hold [T x V] logits; an MI355X holds them outright
// (512 x 152064 fp32 is 311 MB of 288 GB), so the logits are one hipBLASLt
// GEMM per chunk of up to 2 GB, read twice by one row kernel, and the
// gradient one more GEMM:
//   ce_gather   packs the kept rows of h
//   GEMM        logits [n][V] = h_kept W^T (fp32 results)
//   ce_row      per row: the max and sum of exponentials (one workgroup, each
//               thread online over its strided elements, threads merged in a
//               fixed tree through LDS), lse, the row's loss term and the
//               dlogits softmax - onehot (bf16 in the bf16 mode)
//   GEMM        dh_kept = (1/n) dlogits W
//   ce_scatter  dh rows back in place, zeros for dropped rows
//   ce_loss     the mean of the row terms (double, fixed order)
// Every sum has a fixed order and hipBLASLt runs without workspace, so
// results are bitwise repeatable.
#include <cfloat>

#include "attn_common.hpp"
#include "blas_lt.hpp"
#include "lmhead_launch.hpp"

namespace glacier {
namespace {

constexpr int kCeThreads = 256;

// hv[i] = hidden[rows[r0 + i]], 16-byte pieces (H % 8 == 0).
template <typename IO>
__global__ __launch_bounds__(256) void ce_gather_kernel(const IO* __restrict__ hidden,
                                                        const int* __restrict__ rows, int r0, int n,
                                                        int H, IO* __restrict__ hv) {
  const int per_row = H * (int)sizeof(IO) / 16;
  const long idx = (long)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (long)n * per_row) return;
  const int i = (int)(idx / per_row), p = (int)(idx % per_row);
  const int4* src = reinterpret_cast<const int4*>(hidden + (long)rows[r0 + i] * H);
  reinterpret_cast<int4*>(hv + (long)i * H)[p] = src[p];
}

__device__ inline void merge(float& m, float& s, float m2, float s2) {
  const float mm = fmaxf(m, m2);
  s = s * expf(m - mm) + s2 * expf(m2 - mm);
  m = mm;
}

// One workgroup per kept row r of the chunk (global kept index r0 + r).
// In the fp32 mode dl is the logits buffer itself (no __restrict__): each
// thread rewrites only the pieces it has read, and the target logit is read
// before any rewrite.
template <typename DL>
__global__ __launch_bounds__(kCeThreads) void ce_row_kernel(const float* logits, DL* dl,
                                                            const int* __restrict__ targets, int r0,
                                                            int V, int ldl, int want_grad,
                                                            float* __restrict__ row_loss) {
  __shared__ float sm[kCeThreads], ss[kCeThreads];
  const int r = blockIdx.x, tid = threadIdx.x;
  const float* l = logits + (long)r * ldl;
  const int nq = ldl / 4;
  const int tgt = targets[r0 + r];
  const float tl = tid == 0 ? l[tgt] : 0.0f;
  // each thread: online max and sum over its 4-element pieces tid, tid + 256, ...
  float m = -FLT_MAX, s = 0.0f;
  for (int q = tid; q < nq; q += kCeThreads) {
    const float4 v4 = reinterpret_cast<const float4*>(l)[q];
    const float v[4] = {v4.x, v4.y, v4.z, v4.w};
    float x[4];
    float mq = -FLT_MAX;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      x[e] = 4 * q + e < V ? v[e] : -INFINITY;  // the row's padding is not written
      mq = fmaxf(mq, x[e]);
    }
    const float mn = fmaxf(m, mq);
    float t = 0.0f;
#pragma unroll
    for (int e = 0; e < 4; ++e) t += expf(x[e] - mn);
    s = s * expf(m - mn) + t;
    m = mn;
  }
  sm[tid] = m;
  ss[tid] = s;
  __syncthreads();
  for (int w = kCeThreads / 2; w > 0; w /= 2) {
    if (tid < w) {
      float a = sm[tid], b = ss[tid];
      merge(a, b, sm[tid + w], ss[tid + w]);
      sm[tid] = a;
      ss[tid] = b;
    }
    __syncthreads();
  }
  const float lse = sm[0] + logf(ss[0]);
  if (tid == 0) row_loss[r0 + r] = lse - tl;
  if (!want_grad) return;
  // dlogits = softmax - onehot (each row written by its own workgroup only)
  for (int q = tid; q < nq; q += kCeThreads) {
    const float4 v4 = reinterpret_cast<const float4*>(l)[q];
    const float v[4] = {v4.x, v4.y, v4.z, v4.w};
    f32x4 d;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int j = 4 * q + e;
      d[e] = j < V ? expf(v[e] - lse) - (j == tgt ? 1.0f : 0.0f) : 0.0f;
    }
    store4(dl + (long)r * ldl + 4 * q, d);
  }
}

// d_hidden[t] = dhv[src_of[t]], or zero where src_of[t] < 0; 4 per thread.
template <typename IO>
__global__ __launch_bounds__(256) void ce_scatter_kernel(const float* __restrict__ dhv,
                                                         const int* __restrict__ src_of, int T,
                                                         int H, IO* __restrict__ d_hidden) {
  const long idx = (long)blockIdx.x * 256 + threadIdx.x;
  const int q4 = H / 4;
  if (idx >= (long)T * q4) return;
  const int t = (int)(idx / q4), c = 4 * (int)(idx % q4);
  const int src = src_of[t];
  f32x4 v = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  if (src >= 0) v = *reinterpret_cast<const f32x4*>(dhv + (long)src * H + c);
  store4(d_hidden + (long)t * H + c, v);
}

// loss = (float)(sum_r row_loss[r] * (1/n)), the sum in double in a fixed
// order (one workgroup).
__global__ __launch_bounds__(256) void ce_loss_kernel(const float* __restrict__ row_loss, int n,
                                                      float* __restrict__ loss) {
  __shared__ double part[256];
  double acc = 0.0;
  for (int i = threadIdx.x; i < n; i += 256) acc += (double)row_loss[i];
  part[threadIdx.x] = acc;
  __syncthreads();
  for (int w = 128; w > 0; w /= 2) {
    if ((int)threadIdx.x < w) part[threadIdx.x] += part[threadIdx.x + w];
    __syncthreads();
  }
  if (threadIdx.x == 0) loss[0] = (float)(part[0] * (double)(1.0f / (float)n));
}

unsigned blocks(long n, int per) { return static_cast<unsigned>((n + per - 1) / per); }

template <typename IO>
hipError_t run(const LmHeadLaunch& a, hipStream_t st, void* blas) {
  constexpr bool BF = sizeof(IO) == 2;
  const bool grad = a.d_hidden != nullptr;
  const int per_row = a.H * (int)sizeof(IO) / 16;
  for (int r0 = 0; r0 < a.n_valid; r0 += a.chunk) {
    const int n = std::min(a.chunk, a.n_valid - r0);
    hipLaunchKernelGGL(ce_gather_kernel<IO>, dim3(blocks((long)n * per_row, 256)), dim3(256), 0, st,
                       static_cast<const IO*>(a.hidden), a.rows, r0, n, a.H, static_cast<IO*>(a.hv));
    GL_CHECK(hipGetLastError());
    GL_CHECK(blas_gemm(blas, BF, false, true, n, a.V, a.H, 1.0f, a.hv, a.H, a.weight, a.H, 0.0f,
                       a.logits, a.ldl, st));
    hipLaunchKernelGGL(ce_row_kernel<IO>, dim3(n), dim3(kCeThreads), 0, st, a.logits,
                       static_cast<IO*>(a.dl), a.targets, r0, a.V, a.ldl, grad ? 1 : 0, a.row_loss);
    GL_CHECK(hipGetLastError());
    if (grad)
      GL_CHECK(blas_gemm(blas, BF, false, false, n, a.H, a.V, 1.0f / (float)a.n_valid, a.dl, a.ldl,
                         a.weight, a.H, 0.0f, a.dhv + (long)r0 * a.H, a.H, st));
  }
  if (grad) {
    const long n4 = (long)a.T * (a.H / 4);
    hipLaunchKernelGGL(ce_scatter_kernel<IO>, dim3(blocks(n4, 256)), dim3(256), 0, st, a.dhv,
                       a.src_of, a.T, a.H, static_cast<IO*>(a.d_hidden));
    GL_CHECK(hipGetLastError());
  }
  if (a.n_valid > 0) {
    hipLaunchKernelGGL(ce_loss_kernel, dim3(1), dim3(256), 0, st, a.row_loss, a.n_valid, a.loss);
    GL_CHECK(hipGetLastError());
  }
  return hipSuccess;
}

}  // namespace

hipError_t launch_lmhead(const LmHeadLaunch& a, hipStream_t st, void* blas) {
  return a.io_bf16 ? run<bf16>(a, st, blas) : run<float>(a, st, blas);
}

}  // namespace glacier
