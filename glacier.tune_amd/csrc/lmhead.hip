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
#include <algorithm>
#include <cfloat>

#include "attn_common.hpp"
#include "blas_lt.hpp"
#include "lmhead_launch.hpp"

namespace glacier {
namespace {

// hv[i] = hidden[rows[r0 + i]], 16-byte pieces (H % 8 == 0).
template <typename IO>
__global__ __launch_bounds__(256) void ce_gather_kernel(const IO* __restrict__ hidden,
                                                        const int* __restrict__ rows, int r0, int n,
                                                        int H, IO* __restrict__ hv) {
  const int per_row = ce_gather_pieces(H, (int)sizeof(IO));
  const long idx = (long)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (long)n * per_row) return;
  const CeGatherAt at = ce_gather_at(idx, per_row);
  const int4* src = reinterpret_cast<const int4*>(hidden + (long)rows[r0 + at.i] * H);
  reinterpret_cast<int4*>(hv + (long)at.i * H)[at.p] = src[at.p];
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
  const CeScatterAt at = ce_scatter_at(idx, q4);
  const int t = at.t, c = at.c;
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
  const int per_row = ce_gather_pieces(a.H, (int)sizeof(IO));
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

void lmhead_rows(const int32_t* targets, int T, int V, std::vector<int>& rows,
                 std::vector<int>& tgts, std::vector<int>& src_of) {
  rows.clear();
  tgts.clear();
  src_of.assign(static_cast<size_t>(T), -1);
  for (int t = 0; t < T; ++t) {
    if (targets[t] >= 0 && targets[t] < V) {
      src_of[t] = static_cast<int>(rows.size());
      rows.push_back(t);
      tgts.push_back(targets[t]);
    }
  }
}

void lmhead_shape(LmHeadLaunch& a, int n_valid) {
  a.n_valid = n_valid;
  a.ldl = (a.V + 7) / 8 * 8;
  const long per_row = (long)a.ldl * (4 + (a.io_bf16 ? 2 : 0));
  a.chunk = static_cast<int>(std::max(1L, std::min<long>(n_valid, kLmHeadChunkBytes / per_row)));
}

LmHeadScratch lmhead_scratch(const LmHeadLaunch& a) {
  const size_t esz = a.io_bf16 ? 2 : 4, n = static_cast<size_t>(a.n_valid);
  LmHeadScratch s{};
  s.idx = (2 * n + static_cast<size_t>(a.T)) * sizeof(int);
  if (n > 0) {
    s.hv = static_cast<size_t>(a.chunk) * a.H * esz;
    s.logits = static_cast<size_t>(a.chunk) * a.ldl * 4;
    s.dl = a.io_bf16 ? static_cast<size_t>(a.chunk) * a.ldl * 2 : 0;
    s.dhv = a.d_hidden != nullptr ? n * a.H * 4 : 0;
    s.row_loss = (n + 1) * 4;
  }
  return s;
}

std::string lmhead_check_bounds(const LmHeadLaunch& a, const LmHeadScratch& s, const int* rows,
                                const int* targets, const int* src_of, size_t hidden_elems,
                                size_t weight_elems, size_t d_hidden_elems) {
  const int esz = a.io_bf16 ? 2 : 4;
  const bool grad = a.d_hidden != nullptr;
  const long long hv_elems = s.hv / esz, logit_elems = s.logits / 4, dhv_elems = s.dhv / 4;
  // dlogits: bf16 scratch, or the logits buffer itself in the fp32 mode
  const long long dl_elems = a.io_bf16 ? (long long)(s.dl / 2) : logit_elems;
  auto bad = [](const std::string& what, long long at, long long limit) {
    return what + ": element " + std::to_string(at) + " of " + std::to_string(limit);
  };
  if (s.idx < (2 * (size_t)a.n_valid + (size_t)a.T) * sizeof(int)) return "index scratch too small";
  for (int r = 0; r < a.n_valid; ++r) {
    if (rows[r] < 0 || rows[r] >= a.T) return bad("rows[]", rows[r], a.T);
    if (targets[r] < 0 || targets[r] >= a.V) return bad("targets[]", targets[r], a.V);
  }
  for (int t = 0; t < a.T; ++t)
    if (src_of[t] < -1 || src_of[t] >= a.n_valid) return bad("src_of[]", src_of[t], a.n_valid);
  const int per_row = ce_gather_pieces(a.H, esz), piece = 16 / esz;
  for (int r0 = 0; r0 < a.n_valid; r0 += a.chunk) {
    const int n = std::min(a.chunk, a.n_valid - r0);
    // ce_gather: every thread of its grid
    const long threads = (long)((n * (long)per_row + 255) / 256) * 256;
    for (long idx = 0; idx < threads; ++idx) {
      if (idx >= (long)n * per_row) continue;  // the kernel's early return
      const CeGatherAt at = ce_gather_at(idx, per_row);
      if (r0 + at.i >= a.n_valid) return bad("ce_gather rows[]", r0 + at.i, a.n_valid);
      const long long src = (long long)rows[r0 + at.i] * a.H + (long long)at.p * piece + piece;
      if (src > (long long)hidden_elems) return bad("ce_gather hidden", src, hidden_elems);
      const long long dst = (long long)at.i * a.H + (long long)at.p * piece + piece;
      if (dst > hv_elems) return bad("ce_gather hv", dst, hv_elems);
    }
    // logits GEMM: [n x V] = hv [n x H] . weight[V x H]^T
    const GemmLayouts g1 = gemm_layouts(false, true, n, a.V, a.H, a.H, a.H, a.ldl);
    if (g1.b_first.elements() > (long long)weight_elems)
      return bad("logits GEMM weight", g1.b_first.elements(), weight_elems);
    if (g1.a_second.elements() > hv_elems) return bad("logits GEMM hv", g1.a_second.elements(), hv_elems);
    if (g1.c.elements() > logit_elems) return bad("logits GEMM logits", g1.c.elements(), logit_elems);
    // ce_row: n workgroups of kCeThreads, each thread its quads tid, tid + 256, ...
    const int nq = a.ldl / 4;
    for (int r = 0; r < n; ++r) {
      const long long base = (long long)r * a.ldl;
      if (base + targets[r0 + r] >= logit_elems) return bad("ce_row target logit", base + targets[r0 + r], logit_elems);
      if (r0 + r >= a.n_valid) return bad("ce_row row_loss", r0 + r, a.n_valid);
      for (int tid = 0; tid < kCeThreads; ++tid)
        for (int q = tid; q < nq; q += kCeThreads) {
          const long long end = base + 4LL * q + 4;
          if (end > logit_elems) return bad("ce_row logits", end, logit_elems);
          if (grad && end > dl_elems) return bad("ce_row dlogits", end, dl_elems);
        }
    }
    if (grad) {
      // gradient GEMM: dhv[r0 ..][n x H] = dl [n x V] . weight [V x H]
      const GemmLayouts g2 = gemm_layouts(false, false, n, a.H, a.V, a.ldl, a.H, a.H);
      if (g2.b_first.elements() > (long long)weight_elems)
        return bad("gradient GEMM weight", g2.b_first.elements(), weight_elems);
      if (g2.a_second.elements() > dl_elems) return bad("gradient GEMM dlogits", g2.a_second.elements(), dl_elems);
      const long long c_end = (long long)r0 * a.H + g2.c.elements();
      if (c_end > dhv_elems) return bad("gradient GEMM dhv", c_end, dhv_elems);
    }
  }
  if (grad) {
    // ce_scatter: every thread of its grid
    const int q4 = a.H / 4;
    const long threads = ((long)a.T * q4 + 255) / 256 * 256;
    for (long idx = 0; idx < threads; ++idx) {
      if (idx >= (long)a.T * q4) continue;
      const CeScatterAt at = ce_scatter_at(idx, q4);
      const int src = src_of[at.t];
      if (src >= 0 && (long long)src * a.H + at.c + 4 > dhv_elems)
        return bad("ce_scatter dhv", (long long)src * a.H + at.c + 4, dhv_elems);
      if ((long long)at.t * a.H + at.c + 4 > (long long)d_hidden_elems)
        return bad("ce_scatter d_hidden", (long long)at.t * a.H + at.c + 4, d_hidden_elems);
    }
  }
  // ce_loss reads n_valid row terms and writes the one after them
  if (a.n_valid > 0 && (size_t)(a.n_valid + 1) * 4 > s.row_loss)
    return bad("ce_loss", a.n_valid + 1, s.row_loss / 4);
  return "";
}

}  // namespace glacier
