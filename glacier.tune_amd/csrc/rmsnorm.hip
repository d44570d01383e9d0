// rmsnorm.hip -- the residual add and RMSNorm either side of the attention
// sub-block, forward and backward, on device tensors:
//   forward   x1 = x + delta,  y = (x1 r) w,  r = 1 / sqrt(mean x1^2 + eps)
//   backward  dx = r (w dy) - (r^3 / n) x sum_i (w_i dy_i) x_i + d_residual,
//             d_weight += sum over rows of dy (x r)
// (ElementwiseKernels.RMSNorm / RMSNormBackward and TensorOps.Add of the
// absent Glacier.Tensor 1.1.0 package, called at TransformerBlock.cs:318,
// :505-506, :524, :579, :672, :677, :827, :836 and, per head, :751, :759).
//
// One wave per row: every lane takes the 4-element chunks lane, lane + 64, ...
// of the row, so the row's sums are one fixed-order wave reduction (no LDS, no
// barrier) and the results are bitwise repeatable.  All of a row's loads are
// issued before any is used, at clamped in-bounds addresses (a load under a
// condition would make the wave wait for each in turn); out-of-range chunks
// are zeroed and not stored.  Each lane reads a chunk before it writes the same
// chunk, so y may alias x or delta, and dx may alias dy or d_residual.
// HBM-bound: one read of each input row and one write of each output row.
#include <hip/hip_ext.h>

#include "attn_common.hpp"
#include "norm_launch.hpp"

namespace glacier {
namespace {

constexpr int kNormThreads = 256;  // at most 4 rows (waves) per workgroup

template <typename IO>
struct Raw4;
template <>
struct Raw4<float> {
  using T = float4;
};
template <>
struct Raw4<bf16> {
  using T = bf16x4;
};

template <typename IO>
__device__ inline typename Raw4<IO>::T ld4(const IO* p) {
  return *reinterpret_cast<const typename Raw4<IO>::T*>(p);
}
__device__ inline void cvt4(float4 r, float (&x)[4]) {
  x[0] = r.x; x[1] = r.y; x[2] = r.z; x[3] = r.w;
}
__device__ inline void cvt4(bf16x4 r, float (&x)[4]) {
#pragma unroll
  for (int e = 0; e < 4; ++e) x[e] = (float)r[e];
}

// The value as stored in the io dtype (x1 is normalised as it is stored, so
// that the backward, which reads the stored x1, sees the same row).
template <typename IO>
__device__ inline float as_stored(float v) {
  return to_f32(from_f32<IO>(v));
}

// Sum over the 64 lanes of a wave in a fixed order (every lane gets it).
__device__ inline float wave_sum(float v) {
  v = lanes_sum<32>(v);
  return v + __shfl_xor(v, 32);
}

// CPL: 4-element chunks per lane (n <= 256 CPL).
template <typename IO, int CPL>
__global__ __launch_bounds__(kNormThreads) void rmsnorm_fwd_kernel(NormFwd a) {
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int row = blockIdx.x * (blockDim.x >> 6) + wave;
  if (row >= a.rows) return;
  const int nc = a.n / 4;
  const long base = (long)row * a.n;
  const IO* x = static_cast<const IO*>(a.x) + base;
  const IO* dl = a.delta != nullptr ? static_cast<const IO*>(a.delta) + base : nullptr;
  typename Raw4<IO>::T xr[CPL], dr[CPL];
  float4 wr[CPL];
#pragma unroll
  for (int k = 0; k < CPL; ++k) {
    const int c = min(lane + 64 * k, nc - 1);
    xr[k] = ld4(x + 4 * c);
    wr[k] = *reinterpret_cast<const float4*>(a.w + 4 * c);
  }
  if (dl != nullptr) {
#pragma unroll
    for (int k = 0; k < CPL; ++k) dr[k] = ld4(dl + 4 * min(lane + 64 * k, nc - 1));
  }
  float v[CPL][4];
  float ss = 0.0f;
#pragma unroll
  for (int k = 0; k < CPL; ++k) {
    const bool ok = lane + 64 * k < nc;
    cvt4(xr[k], v[k]);
    if (dl != nullptr) {
      float d[4];
      cvt4(dr[k], d);
#pragma unroll
      for (int e = 0; e < 4; ++e) v[k][e] = as_stored<IO>(v[k][e] + d[e]);
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      v[k][e] = ok ? v[k][e] : 0.0f;
      ss += v[k][e] * v[k][e];
    }
  }
  ss = wave_sum(ss);
  const float r = 1.0f / sqrtf(ss / (float)a.n + a.eps);
  IO* y = static_cast<IO*>(a.y) + base;
  IO* x1 = (dl != nullptr && a.x1 != nullptr) ? static_cast<IO*>(a.x1) + base : nullptr;
#pragma unroll
  for (int k = 0; k < CPL; ++k) {
    const int c = lane + 64 * k;
    if (c >= nc) break;
    float w[4];
    cvt4(wr[k], w);
    f32x4 o;
#pragma unroll
    for (int e = 0; e < 4; ++e) o[e] = (v[k][e] * r) * w[e];
    store4(y + 4 * c, o);
    if (x1 != nullptr) store4(x1 + 4 * c, f32x4{v[k][0], v[k][1], v[k][2], v[k][3]});
  }
}

template <typename IO, int CPL>
__global__ __launch_bounds__(kNormThreads) void rmsnorm_bwd_kernel(NormBwd a) {
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int row = blockIdx.x * (blockDim.x >> 6) + wave;
  if (row >= a.rows) return;
  const int nc = a.n / 4;
  const long base = (long)row * a.n;
  const IO* x = static_cast<const IO*>(a.x) + base;
  const IO* dy = static_cast<const IO*>(a.dy) + base;
  const IO* dres = a.d_residual != nullptr ? static_cast<const IO*>(a.d_residual) + base : nullptr;
  typename Raw4<IO>::T xr[CPL], gr[CPL], rr[CPL];
  float4 wr[CPL];
#pragma unroll
  for (int k = 0; k < CPL; ++k) {
    const int c = min(lane + 64 * k, nc - 1);
    xr[k] = ld4(x + 4 * c);
    gr[k] = ld4(dy + 4 * c);
    wr[k] = *reinterpret_cast<const float4*>(a.w + 4 * c);
  }
  if (dres != nullptr) {
#pragma unroll
    for (int k = 0; k < CPL; ++k) rr[k] = ld4(dres + 4 * min(lane + 64 * k, nc - 1));
  }
  float xv[CPL][4], g[CPL][4];  // g = w dy
  float ss = 0.0f, c = 0.0f;
#pragma unroll
  for (int k = 0; k < CPL; ++k) {
    const bool ok = lane + 64 * k < nc;
    float w[4], d[4];
    cvt4(xr[k], xv[k]);
    cvt4(gr[k], d);
    cvt4(wr[k], w);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      xv[k][e] = ok ? xv[k][e] : 0.0f;
      g[k][e] = ok ? w[e] * d[e] : 0.0f;
      ss += xv[k][e] * xv[k][e];
      c += g[k][e] * xv[k][e];
    }
  }
  ss = wave_sum(ss);
  c = wave_sum(c);
  const float r = 1.0f / sqrtf(ss / (float)a.n + a.eps);
  const float kx = r * r * r / (float)a.n * c;
  IO* dx = static_cast<IO*>(a.dx) + base;
#pragma unroll
  for (int k = 0; k < CPL; ++k) {
    const int ci = lane + 64 * k;
    if (ci >= nc) break;
    float res[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (dres != nullptr) cvt4(rr[k], res);
    f32x4 o;
#pragma unroll
    for (int e = 0; e < 4; ++e) o[e] = (r * g[k][e] - kx * xv[k][e]) + res[e];
    store4(dx + 4 * ci, o);
  }
  if (a.rstd != nullptr && lane == 0) a.rstd[row] = r;
}

// d_weight[i] += sum over rows t (ascending) of dy[t][i] (x[t][i] r[t]); one
// column per thread, the rows unrolled by 8 so that their loads overlap.
template <typename IO>
__global__ __launch_bounds__(256) void rmsnorm_dw_kernel(NormBwd a) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i >= a.n) return;
  const IO* x = static_cast<const IO*>(a.x) + i;
  const IO* dy = static_cast<const IO*>(a.dy_w) + i;  // dy as passed in, even when dx overwrote it
  float acc = 0.0f;
  int t = 0;
  for (; t + 8 <= a.rows; t += 8) {
    float xs[8], ds[8], rs[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      xs[u] = to_f32(x[(long)(t + u) * a.n]);
      ds[u] = to_f32(dy[(long)(t + u) * a.n]);
      rs[u] = a.rstd[t + u];
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) acc += ds[u] * (xs[u] * rs[u]);
  }
  for (; t < a.rows; ++t) acc += to_f32(dy[(long)t * a.n]) * (to_f32(x[(long)t * a.n]) * a.rstd[t]);
  a.d_weight[i] += acc;
}

unsigned blocks(long n, int per) { return static_cast<unsigned>((n + per - 1) / per); }

// Rows (waves) per workgroup: one for short calls, so that a 512-row call
// has 512 workgroups for the 256 CUs; up to four for long ones
// (measured on MI355X: 512 x 3584 bf16 fwd 5.3 us at 1, 6.0 us at 4; 14336 x
// 128 5.7 us at 4, 6.4 us at 1).
int rows_per_workgroup(int rows) { return rows >= 4096 ? 4 : rows >= 2048 ? 2 : 1; }

// Chunks per lane, rounded up to the instantiated sizes.
int chunks_per_lane(int n) {
  const int need = (n / 4 + 63) / 64;
  int cpl = 1;
  while (cpl < need) cpl *= 2;
  return cpl;
}

template <typename IO>
hipError_t fwd(const NormFwd& a, hipStream_t st, KernelTimer* tm) {
  const int rpw = rows_per_workgroup(a.rows);
  const dim3 grid(blocks(a.rows, rpw)), block(64 * rpw);
  LaunchTiming t(tm, kKernNormFwd);
  switch (chunks_per_lane(a.n)) {
#define GL_NORM(C)                                                                              \
  GL_LAUNCH(t, (rmsnorm_fwd_kernel<IO, C>), grid, block, 0, st, \
                        a)
    case 1: GL_NORM(1); break;
    case 2: GL_NORM(2); break;
    case 4: GL_NORM(4); break;
    case 8: GL_NORM(8); break;
    case 16: GL_NORM(16); break;
    case 32: GL_NORM(32); break;
#undef GL_NORM
    default: return hipErrorInvalidValue;
  }
  GL_CHECK(hipGetLastError());
  t.launched();
  return hipSuccess;
}

template <typename IO>
hipError_t bwd(const NormBwd& a, hipStream_t st, KernelTimer* tm) {
  const int rpw = rows_per_workgroup(a.rows);
  const dim3 grid(blocks(a.rows, rpw)), block(64 * rpw);
  {
    LaunchTiming t(tm, kKernNormBwd);
    switch (chunks_per_lane(a.n)) {
#define GL_NORM(C)                                                                              \
  GL_LAUNCH(t, (rmsnorm_bwd_kernel<IO, C>), grid, block, 0, st, \
                        a)
      case 1: GL_NORM(1); break;
      case 2: GL_NORM(2); break;
      case 4: GL_NORM(4); break;
      case 8: GL_NORM(8); break;
      case 16: GL_NORM(16); break;
      case 32: GL_NORM(32); break;
#undef GL_NORM
      default: return hipErrorInvalidValue;
    }
    GL_CHECK(hipGetLastError());
    t.launched();
  }
  if (a.d_weight != nullptr) {
    hipLaunchKernelGGL(rmsnorm_dw_kernel<IO>, dim3(blocks(a.n, 256)), dim3(256), 0, st, a);
    GL_CHECK(hipGetLastError());
  }
  return hipSuccess;
}

}  // namespace

hipError_t launch_rmsnorm_forward(const NormFwd& a, hipStream_t st, KernelTimer* tm) {
  return a.io_bf16 ? fwd<bf16>(a, st, tm) : fwd<float>(a, st, tm);
}

hipError_t launch_rmsnorm_backward(const NormBwd& a, hipStream_t st, KernelTimer* tm) {
  return a.io_bf16 ? bwd<bf16>(a, st, tm) : bwd<float>(a, st, tm);
}

}  // namespace glacier
