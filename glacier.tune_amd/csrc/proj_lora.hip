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
//
// The base products X W_p^T and dY_p W_p are GEMMs with fp32 results, all on
// the library's own kernels (proj_gemm.hip): for bf16 tensors the narrow
// GEMM (the k and v projections of a GQA block) and the wide one (q), and
// for fp32 tensors or shapes neither takes, a generic fp32-MFMA GEMM.
// Everything low-rank is here, each kernel taking every projection of the
// call in one launch:
//   lowrank_rows    L = X A_p and dL = dY_p B_p^T (output r columns wide,
//                   reduction over in / out): 16-row slabs, the reduction
//                   split over workgroups and over their 8 waves, fp32 MFMAs
//   lowrank_reduce  adds the workgroups' split sums in split order
//   lowrank_cols    grad_A += s X^T dL, grad_B += s L^T dY (reduction over
//                   the tokens): 64-column slabs, tokens split over 8 waves
//   lowrank_out     Y_p = io(Yf_p + bias_p + (s L) B_p) and dX = io(dXf +
//                   sum_p (s dL_p) A_p^T): 16 x 256 tiles, the rank-r
//                   product on MFMAs, fused with the dtype conversion
// The adapters, the low-rank activations and the gradients stay fp32, as in
// the reference (LoraAdapter.cs:23-24); bf16 tensors round only the base
// operands and the outputs.  Every reduction has a fixed order, so every
// result is bitwise repeatable.
#include "attn_common.hpp"
#include "proj_launch.hpp"

namespace glacier {
namespace {

constexpr int kLrWaves = 8;  // waves of a rows/cols workgroup, splitting the reduction
constexpr int kLrThreads = 64 * kLrWaves;
constexpr int kOutThreads = 256;  // lowrank_out: 4 waves of 16 x 64
constexpr int kMaxJobs = 2 * kMaxProj;

__device__ inline void load4(const float* p, float (&x)[4]) {
  const float4 a = *reinterpret_cast<const float4*>(p);
  x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w;
}

// 4 consecutive elements as loaded, converted (or zeroed) only when used:
// every load of a step is issued at an in-bounds (clamped) address before any
// value is used, and out-of-range values of ONE operand of each product are
// zeroed afterwards; the other operand's clamped values then meet zeros, or
// reach only outputs that are not stored.  (A load under a condition makes
// the wave wait for each load in turn; so would a select on both operands,
// which the compiler turns back into conditional loads.)
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
__device__ inline typename Raw4<IO>::T ld_raw4(const IO* p) {
  return *reinterpret_cast<const typename Raw4<IO>::T*>(p);
}
__device__ inline void sel4(float4 r, bool ok, float (&x)[4]) {
  x[0] = ok ? r.x : 0.0f;
  x[1] = ok ? r.y : 0.0f;
  x[2] = ok ? r.z : 0.0f;
  x[3] = ok ? r.w : 0.0f;
}
__device__ inline void sel4(bf16x4 r, bool ok, float (&x)[4]) {
#pragma unroll
  for (int e = 0; e < 4; ++e) x[e] = ok ? (float)r[e] : 0.0f;
}

__device__ inline f32x4 mma_f32(float a, float b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// The [lo, hi) share of part p of n of a range [0, len), cut at multiples of g.
__device__ inline void share(int len, int n, int p, int g, int& lo, int& hi) {
  const int per = (len + n * g - 1) / (n * g) * g;
  lo = min(len, p * per);
  hi = min(len, lo + per);
}

// One product Out [T][r] = U [T][K] V of lowrank_rows: V = A [K][r] (vt 0)
// or B^T with B [r][K] (vt 1); U in the call's dtype.
struct RowsJob {
  const void* u;
  const float* v;
  int K;
  int vt;
};
struct RowsJobs {
  RowsJob j[kMaxJobs];
};

// The k range [kb, ke) of one wave of lowrank_rows_kernel, added into acc.
// In a step of 16 lane (i = lane % 16, q = lane / 16) loads U[row i][k0 + 4q
// .. +4] and, for MFMA e of the step, supplies U[i][k0 + 4q + e] and V(k0 +
// 4q + e, 16 jt + i): each MFMA's reduction index q maps to one k for both
// operands.  U is zeroed for k past the slice and for rows >= T.
template <typename IO, int NT, bool VT>
__device__ inline void rows_accumulate(const IO* __restrict__ urow, bool row_ok,
                                       const float* __restrict__ v, int K, int rank, int kb, int ke,
                                       f32x4 (&acc)[NT]) {
  constexpr int CH = NT <= 2 ? 8 : 4;  // steps whose loads are issued together
  const int lane = threadIdx.x & 63, i = lane & 15, q = lane >> 4;
  for (int k0 = kb; k0 < ke; k0 += 16 * CH) {
    typename Raw4<IO>::T xr[CH];
    float w[CH][NT][4];
#pragma unroll
    for (int s = 0; s < CH; ++s) {
      if (k0 + 16 * s >= ke) break;  // the wave's slice ends (uniform)
      const int kc = min(k0 + 16 * s + 4 * q, K - 4);  // K % 4 == 0
      xr[s] = ld_raw4(urow + kc);
#pragma unroll
      for (int jt = 0; jt < NT; ++jt) {
        const int jc = min(16 * jt + i, rank - 1);
        if constexpr (VT) {
          const float4 r = *reinterpret_cast<const float4*>(v + (long)jc * K + kc);
          w[s][jt][0] = r.x; w[s][jt][1] = r.y; w[s][jt][2] = r.z; w[s][jt][3] = r.w;
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e) w[s][jt][e] = v[(long)(kc + e) * rank + jc];
        }
      }
    }
#pragma unroll
    for (int s = 0; s < CH; ++s) {
      if (k0 + 16 * s >= ke) break;
      const bool k_ok = k0 + 16 * s + 4 * q < ke;  // a 4-chunk is all in or all out
      float x[4];
      sel4(xr[s], k_ok && row_ok, x);
#pragma unroll
      for (int jt = 0; jt < NT; ++jt)
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[jt] = mma_f32(x[e], w[s][jt][e], acc[jt]);
    }
  }
}

// Workgroup (x, y, z): rows 16x.. of job z, split y of its K; wave w reduces
// a contiguous slice of that split (rows_accumulate).  The workgroup's sums
// (waves added in order through LDS) go to part[z][y][x][16][16 NT].
template <typename IO, int NT>
__global__ __launch_bounds__(kLrThreads) void lowrank_rows_kernel(RowsJobs jobs, int rows, int rank,
                                                                  float* __restrict__ part) {
  constexpr int kOut = 16 * NT * 16;  // outputs of the workgroup
  __shared__ float red[kLrWaves * kOut];
  const RowsJob& job = jobs.j[blockIdx.z];
  const int K = job.K;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int i = lane & 15, q = lane >> 4;
  const int t0 = blockIdx.x * 16;
  const bool row_ok = t0 + i < rows;
  const IO* urow = static_cast<const IO*>(job.u) + (long)(row_ok ? t0 + i : 0) * K;
  int k_lo, k_hi, kb, ke;
  share(K, gridDim.y, blockIdx.y, 16, k_lo, k_hi);
  share(k_hi - k_lo, kLrWaves, wave, 16, kb, ke);
  f32x4 acc[NT];
#pragma unroll
  for (int jt = 0; jt < NT; ++jt) acc[jt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  if (job.vt)
    rows_accumulate<IO, NT, true>(urow, row_ok, job.v, K, rank, k_lo + kb, k_lo + ke, acc);
  else
    rows_accumulate<IO, NT, false>(urow, row_ok, job.v, K, rank, k_lo + kb, k_lo + ke, acc);
  // D of tile jt: lane (i, q), register c holds row 4q + c, column 16 jt + i.
#pragma unroll
  for (int jt = 0; jt < NT; ++jt)
#pragma unroll
    for (int c = 0; c < 4; ++c) red[wave * kOut + (4 * q + c) * (16 * NT) + 16 * jt + i] = acc[jt][c];
  __syncthreads();
  float* mine = part + (((long)blockIdx.z * gridDim.y + blockIdx.y) * gridDim.x + blockIdx.x) * kOut;
  for (int idx = threadIdx.x; idx < kOut; idx += kLrThreads) {
    float sum = 0.0f;
#pragma unroll
    for (int wv = 0; wv < kLrWaves; ++wv) sum += red[wv * kOut + idx];
    mine[idx] = sum;
  }
}

// dense[z][t][j] = sum over the splits s (ascending) of part[z][s][t / 16]
// [t % 16][j], for every job z of a lowrank_rows launch.
__global__ __launch_bounds__(256) void lowrank_reduce_kernel(const float* __restrict__ part,
                                                             float* __restrict__ dense, int n_jobs,
                                                             int splits, int slabs, int width,
                                                             int T, int rank) {
  const long idx = (long)blockIdx.x * 256 + threadIdx.x;
  const long per_job = (long)T * rank;
  if (idx >= n_jobs * per_job) return;
  const int z = (int)(idx / per_job), t = (int)(idx % per_job / rank), j = (int)(idx % rank);
  const long slab_floats = 16L * width;
  const float* p = part + ((long)z * splits * slabs + t / 16) * slab_floats + (t % 16) * width + j;
  float sum = 0.0f;
  for (int s = 0; s < splits; ++s) sum += p[(long)s * slabs * slab_floats];
  dense[idx] = sum;
}

// One product Out (+)= alpha U^T W of lowrank_cols: U [T][cols] in the call's
// dtype, W [T][r] fp32; Out [cols][r] or, transposed, [r][cols];
// workgroups first .. first + ceil(cols / 64) - 1.
struct ColsJob {
  const void* u;
  const float* w;
  float* out;
  int cols;
  float alpha;
  int transposed;
  int first;
};
struct ColsJobs {
  ColsJob j[kMaxJobs];
  int n;
};

// Workgroup: 64 columns of one job; wave w reduces a contiguous slice of the
// tokens in steps of 4.  Lane (i, q) loads U[t0 + q][c0 + 4i .. +4]: element
// e feeds tile e, whose row i is column c0 + 4i + e, with W[t0 + q][16 jt +
// i] as the other operand.  The waves' sums are added in order through LDS.
template <typename IO, int NT>
__global__ __launch_bounds__(kLrThreads) void lowrank_cols_kernel(ColsJobs jobs, int T, int rank) {
  constexpr int CH = 8;
  constexpr int kPad = 17;  // LDS row stride: the 4 lane groups fall in different banks
  __shared__ float red[kLrWaves * 64 * kPad];
  int z = 0;
  while (z + 1 < jobs.n && (int)blockIdx.x >= jobs.j[z + 1].first) ++z;
  const ColsJob& job = jobs.j[z];
  const IO* u = static_cast<const IO*>(job.u);
  const float* w = job.w;
  const int cols = job.cols;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int i = lane & 15, q = lane >> 4;
  const int c0 = ((int)blockIdx.x - job.first) * 64;
  const bool col_ok = c0 + 4 * i < cols;  // cols % 4 == 0
  int tb, te;
  share(T, kLrWaves, wave, 4, tb, te);
  f32x4 acc[4][NT];
#pragma unroll
  for (int e = 0; e < 4; ++e)
#pragma unroll
    for (int jt = 0; jt < NT; ++jt) acc[e][jt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  const IO* ucol = u + min(c0 + 4 * i, cols - 4);
  for (int t0 = tb; t0 < te; t0 += 4 * CH) {
    typename Raw4<IO>::T xr[CH];
    float wv[CH][NT];
#pragma unroll
    for (int s = 0; s < CH; ++s) {
      if (t0 + 4 * s >= te) break;  // the wave's slice ends (uniform)
      const int tc = min(t0 + 4 * s + q, T - 1);
      xr[s] = ld_raw4(ucol + (long)tc * cols);
#pragma unroll
      for (int jt = 0; jt < NT; ++jt) wv[s][jt] = w[(long)tc * rank + min(16 * jt + i, rank - 1)];
    }
#pragma unroll
    for (int s = 0; s < CH; ++s) {
      if (t0 + 4 * s >= te) break;
      const bool t_ok = t0 + 4 * s + q < te;
      float x[4];
      sel4(xr[s], t_ok && col_ok, x);
#pragma unroll
      for (int jt = 0; jt < NT; ++jt)
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[e][jt] = mma_f32(x[e], wv[s][jt], acc[e][jt]);
    }
  }
  // D of tile (e, jt): lane (i, q), register c holds column c0 + 4 (4q + c) +
  // e, rank 16 jt + i.  One rank tile at a time through LDS.
#pragma unroll
  for (int jt = 0; jt < NT; ++jt) {
    if (jt > 0) __syncthreads();
#pragma unroll
    for (int e = 0; e < 4; ++e)
#pragma unroll
      for (int c = 0; c < 4; ++c) red[(wave * 64 + 4 * (4 * q + c) + e) * kPad + i] = acc[e][jt][c];
    __syncthreads();
    for (int idx = threadIdx.x; idx < 64 * 16; idx += kLrThreads) {
      // transposed output: consecutive threads take consecutive columns
      const int cl = job.transposed ? idx % 64 : idx / 16, jl = job.transposed ? idx / 64 : idx % 16;
      float sum = 0.0f;
#pragma unroll
      for (int wv2 = 0; wv2 < kLrWaves; ++wv2) sum += red[(wv2 * 64 + cl) * kPad + jl];
      const int c = c0 + cl, j = 16 * jt + jl;
      if (c < cols && j < rank) {
        float* o = job.transposed ? job.out + (long)j * cols + c : job.out + (long)c * rank + j;
        *o += job.alpha * sum;
      }
    }
  }
}

// One output of lowrank_out: out [T][n] = io(base [T][n] + bias [n] + sum
// over the terms of (s L [T][r]) V), V = B [r][n] (forward) or A^T with A
// [n][r] (dX); workgroups first .. first + ceil(T / 16) ceil(n / 256) - 1.
struct OutJob {
  const float* base;
  const float* bias;  // or null
  void* out;
  int n;
  int n_terms;
  int first;
  const float* l[kMaxProj];
  const float* v[kMaxProj];
  float s[kMaxProj];
  int nbase = 1;      // base products summed in order: base + i * stride, i < nbase
  long stride = 0;
};
struct OutJobs {
  OutJob j[kMaxProj];
  int n;
};

// Workgroup: 16 tokens x 256 columns of one output, wave w the columns 64w..
// of those.  Lane (i, q) owns columns col = n0 + 4i .. +4: tile e's column i
// is n0 + 4i + e, so that register c of the 4 tiles holds out[t0 + 4q +
// c][col .. col + 4].  In MFMA step m of a group of 16 ranks m0.., the
// reduction index q is rank m0 + 4q + m: a lane's 4 ranks are consecutive,
// one 16-byte load of L, and of A (dX) or of each row of B (forward), when
// r % 4 == 0 (VEC).
template <typename IO, bool AT, bool VEC>
__global__ __launch_bounds__(kOutThreads) void lowrank_out_kernel(OutJobs jobs, int T, int rank) {
  int z = 0;
  while (z + 1 < jobs.n && (int)blockIdx.x >= jobs.j[z + 1].first) ++z;
  const OutJob& job = jobs.j[z];
  const int n = job.n;
  const int b = (int)blockIdx.x - job.first, ncb = (n + 255) / 256;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int i = lane & 15, q = lane >> 4;
  const int t0 = (b / ncb) * 16, col = (b % ncb) * 256 + 64 * wave + 4 * i;
  const bool col_ok = col < n;  // n % 4 == 0
  const int colc = min(col, n - 4);
  f32x4 base[4];
#pragma unroll
  for (int c = 0; c < 4; ++c)
    base[c] = *reinterpret_cast<const f32x4*>(job.base + (long)min(t0 + 4 * q + c, T - 1) * n + colc);
  for (int i = 1; i < job.nbase; ++i) {  // split partials, in order
#pragma unroll
    for (int c = 0; c < 4; ++c)
      base[c] += *reinterpret_cast<const f32x4*>(job.base + i * job.stride +
                                                 (long)min(t0 + 4 * q + c, T - 1) * n + colc);
  }
  f32x4 acc[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) acc[e] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  const bool row_ok = t0 + i < T;
  for (int term = 0; term < job.n_terms; ++term) {
    const float* L = job.l[term] + (long)min(t0 + i, T - 1) * rank;
    const float* V = job.v[term];
    const float s = job.s[term];
    for (int m0 = 0; m0 < rank; m0 += 16) {
      const int jb = m0 + 4 * q;  // this lane's ranks jb .. jb + 3
      float a[4], bv[4][4];       // a[m] = L[t][jb + m], bv[m][e] = V(jb + m, col + e)
      if constexpr (VEC) {  // r % 4 == 0
        const int jc = min(jb, rank - 4);
        load4(L + jc, a);
        if constexpr (AT) {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            float r4[4];
            load4(V + (long)(colc + e) * rank + jc, r4);
#pragma unroll
            for (int m = 0; m < 4; ++m) bv[m][e] = r4[m];
          }
        } else {
#pragma unroll
          for (int m = 0; m < 4; ++m) load4(V + (long)(jc + m) * n + colc, bv[m]);
        }
      } else {
#pragma unroll
        for (int m = 0; m < 4; ++m) {
          const int j = min(jb + m, rank - 1);
          a[m] = L[j];
#pragma unroll
          for (int e = 0; e < 4; ++e) bv[m][e] = AT ? V[(long)(colc + e) * rank + j] : V[(long)j * n + colc + e];
        }
      }
#pragma unroll
      for (int m = 0; m < 4; ++m) a[m] = jb + m < rank && row_ok ? s * a[m] : 0.0f;
#pragma unroll
      for (int m = 0; m < 4; ++m)
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[e] = mma_f32(a[m], bv[m][e], acc[e]);
    }
  }
  if (!col_ok) return;
  f32x4 bias = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  if (job.bias != nullptr) {
#pragma unroll
    for (int e = 0; e < 4; ++e) bias[e] = job.bias[col + e];
  }
  IO* out = static_cast<IO*>(job.out);
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const int t = t0 + 4 * q + c;
    if (t >= T) continue;
    f32x4 y;
#pragma unroll
    for (int e = 0; e < 4; ++e) y[e] = base[c][e] + bias[e] + acc[e][c];
    store4(out + (long)t * n + col, y);
  }
}

unsigned blocks(long n, int per) { return static_cast<unsigned>((n + per - 1) / per); }

// The low-rank products X A_p / dY_p B_p^T of a call: which are needed, and
// where their results go (slot z of ProjLaunch::lowrank, [T][r] each).
struct RowsPlan {
  RowsJobs jobs{};
  int n = 0, kmax = 0;
  int slot_l[kMaxProj], slot_dl[kMaxProj];  // -1: not computed
};

RowsPlan rows_plan(const ProjLaunch& a, bool backward) {
  RowsPlan plan;
  for (int p = 0; p < a.n_proj; ++p) {
    const ProjSpec& s = a.p[p];
    plan.slot_l[p] = plan.slot_dl[p] = -1;
    if (s.a == nullptr) continue;
    if (backward) {
      plan.slot_dl[p] = plan.n;
      plan.jobs.j[plan.n++] = RowsJob{s.dy, s.b, s.out, 1};
      plan.kmax = std::max(plan.kmax, s.out);
    }
    if (!backward || s.grad_b != nullptr) {
      plan.slot_l[p] = plan.n;
      plan.jobs.j[plan.n++] = RowsJob{a.x, s.a, a.in, 0};
      plan.kmax = std::max(plan.kmax, a.in);
    }
  }
  return plan;
}

// Workgroups splitting each reduction of lowrank_rows: about 512 workgroups
// in all, at least 128 reduction elements per split.
int rows_splits(const ProjLaunch& a, const RowsPlan& plan) {
  const int slabs = (a.T + 15) / 16, per = std::max(1, slabs * plan.n);
  return std::max(1, std::min({(512 + per - 1) / per, plan.kmax / 128, 16}));
}

template <typename IO>
hipError_t run_rows(const ProjLaunch& a, const RowsPlan& plan, hipStream_t st) {
  if (plan.n == 0) return hipSuccess;
  const int slabs = (a.T + 15) / 16, splits = rows_splits(a, plan), nt = (a.rank + 15) / 16;
  const dim3 grid(slabs, splits, plan.n), block(kLrThreads);
  switch (nt) {
#define GL_ROWS(NT) \
  hipLaunchKernelGGL((lowrank_rows_kernel<IO, NT>), grid, block, 0, st, plan.jobs, a.T, a.rank, a.part)
    case 1: GL_ROWS(1); break;
    case 2: GL_ROWS(2); break;
    case 3: GL_ROWS(3); break;
    case 4: GL_ROWS(4); break;
#undef GL_ROWS
    default: return hipErrorInvalidValue;
  }
  GL_CHECK(hipGetLastError());
  const long n = (long)plan.n * a.T * a.rank;
  hipLaunchKernelGGL(lowrank_reduce_kernel, dim3(blocks(n, 256)), dim3(256), 0, st, a.part,
                     a.lowrank, plan.n, splits, slabs, 16 * nt, a.T, a.rank);
  return hipGetLastError();
}

template <typename IO, bool AT>
hipError_t run_out(const ProjLaunch& a, OutJobs& jobs, hipStream_t st) {
  int total = 0;
  for (int z = 0; z < jobs.n; ++z) {
    jobs.j[z].first = total;
    total += ((a.T + 15) / 16) * ((jobs.j[z].n + 255) / 256);
  }
  if (a.rank % 4 == 0)
    hipLaunchKernelGGL((lowrank_out_kernel<IO, AT, true>), dim3(total), dim3(kOutThreads), 0, st,
                       jobs, a.T, a.rank);
  else
    hipLaunchKernelGGL((lowrank_out_kernel<IO, AT, false>), dim3(total), dim3(kOutThreads), 0, st,
                       jobs, a.T, a.rank);
  return hipGetLastError();
}

const float* slot(const ProjLaunch& a, int z) { return a.lowrank + (long)z * a.T * a.rank; }

// Which projections of a call take the narrow GEMM, which the wide one; the
// rest (fp32 tensors, shapes neither covers) take the generic one.
bool is_narrow(const ProjLaunch& a, int p) {
  return a.io_bf16 && narrow_gemm_fits(a.in, a.p[p].out);
}
bool is_wide(const ProjLaunch& a, int p) {
  return a.io_bf16 && !is_narrow(a, p) && wide_gemm_fits(a.in, a.p[p].out);
}

// Input slices of the narrow forward launch (1 when there is none).
int fwd_splits(const ProjLaunch& a) {
  int tiles = 0;
  for (int p = 0; p < a.n_proj; ++p)
    if (is_narrow(a, p)) tiles += narrow_feature_tiles(a.p[p].out);
  return tiles == 0 ? 1 : narrow_fwd_splits(a.T, tiles);
}

template <typename IO>
hipError_t forward_impl(const ProjLaunch& a, hipStream_t st) {
  long off = 0;
  OutJobs out{};
  out.n = a.n_proj;
  NarrowFwd nf{};
  nf.x = a.x;
  nf.T = a.T;
  nf.K = a.in;
  nf.nsplit = fwd_splits(a);
  nf.kchunk = (a.in + 64 * nf.nsplit - 1) / (64 * nf.nsplit) * 64;
  for (int p = 0; p < a.n_proj; ++p) {
    const ProjSpec& s = a.p[p];
    out.j[p] = OutJob{a.yf + off, s.bias, s.y, s.out, 0, 0, {}, {}, {}};
    if (is_narrow(a, p)) {
      // Yf_p[i] = X W_p^T over input slice i, summed by lowrank_out
      nf.j[nf.n++] = NarrowJob{s.w, nullptr, a.yf + off, s.out, 0};
      out.j[p].nbase = nf.nsplit;
      out.j[p].stride = (long)a.T * s.out;
      off += (long)nf.nsplit * a.T * s.out;
    } else if (is_wide(a, p)) {
      // Yf_p = X W_p^T on the library's own wide GEMM
      GL_CHECK(launch_wide_fwd(WideFwd{a.x, s.w, a.yf + off, a.T, a.in, s.out}, st));
      off += (long)a.T * s.out;
    } else {
      // Yf_p = X W_p^T on the generic GEMM
      GL_CHECK(launch_generic_fwd(WideFwd{a.x, s.w, a.yf + off, a.T, a.in, s.out}, a.io_bf16, st));
      off += (long)a.T * s.out;
    }
  }
  if (nf.n > 0) GL_CHECK(launch_narrow_fwd(nf, st));
  const RowsPlan plan = rows_plan(a, false);
  GL_CHECK(run_rows<IO>(a, plan, st));  // L_p = X A_p
  for (int p = 0; p < a.n_proj; ++p) {
    if (plan.slot_l[p] < 0) continue;
    OutJob& o = out.j[p];
    o.n_terms = 1;
    o.l[0] = slot(a, plan.slot_l[p]);
    o.v[0] = a.p[p].b;
    o.s[0] = a.p[p].scaling;
  }
  return run_out<IO, false>(a, out, st);  // Y_p = io(Yf_p + bias_p + (s L_p) B_p)
}

template <typename IO>
hipError_t backward_impl(const ProjLaunch& a, hipStream_t st) {
  // dXf = sum_p dY_p W_p: the wide projections (one launch over all of
  // them), then the generic ones (one launch, adding to the wide sum) into
  // dxf, the narrow ones into the buffer after it; lowrank_out adds the two
  NarrowBwd nb{};
  nb.T = a.T;
  nb.K = a.in;
  nb.c = a.dxf + (long)a.T * a.in;
  WideBwd wb{}, gb{};
  wb.c = gb.c = a.dxf;
  wb.T = gb.T = a.T;
  wb.K = gb.K = a.in;
  for (int p = 0; p < a.n_proj; ++p) {
    const ProjSpec& s = a.p[p];
    if (is_narrow(a, p))
      nb.j[nb.n++] = NarrowJob{s.w, s.dy, nullptr, s.out, 0};
    else if (is_wide(a, p))
      wb.j[wb.n++] = WideJob{s.w, s.dy, s.out};
    else
      gb.j[gb.n++] = WideJob{s.w, s.dy, s.out};
  }
  if (wb.n > 0) GL_CHECK(launch_wide_bwd(wb, st));
  gb.accumulate = wb.n > 0;
  if (gb.n > 0) GL_CHECK(launch_generic_bwd(gb, a.io_bf16, st));
  const int wide = wb.n + gb.n;  // products written into dxf
  if (nb.n > 0) GL_CHECK(launch_narrow_bwd(nb, st));
  // dL_p = dY_p B_p^T, and L_p = X A_p where grad_B_p is wanted
  const RowsPlan plan = rows_plan(a, true);
  GL_CHECK(run_rows<IO>(a, plan, st));
  // grad_A_p += s X^T dL_p;  grad_B_p += s L_p^T dY_p
  ColsJobs cj{};
  int total = 0;
  for (int p = 0; p < a.n_proj; ++p) {
    const ProjSpec& s = a.p[p];
    if (s.a == nullptr) continue;
    if (s.grad_a != nullptr) {
      cj.j[cj.n++] = ColsJob{a.x, slot(a, plan.slot_dl[p]), s.grad_a, a.in, s.scaling, 0, total};
      total += (a.in + 63) / 64;
    }
    if (s.grad_b != nullptr) {
      cj.j[cj.n++] = ColsJob{s.dy, slot(a, plan.slot_l[p]), s.grad_b, s.out, s.scaling, 1, total};
      total += (s.out + 63) / 64;
    }
  }
  if (cj.n > 0) {
    switch ((a.rank + 15) / 16) {
#define GL_COLS(NT) \
  hipLaunchKernelGGL((lowrank_cols_kernel<IO, NT>), dim3(total), dim3(kLrThreads), 0, st, cj, a.T, a.rank)
      case 1: GL_COLS(1); break;
      case 2: GL_COLS(2); break;
      case 3: GL_COLS(3); break;
      case 4: GL_COLS(4); break;
#undef GL_COLS
      default: return hipErrorInvalidValue;
    }
    GL_CHECK(hipGetLastError());
  }
  // dX = io(dXf + sum_p (s dL_p) A_p^T)
  OutJobs out{};
  out.n = 1;
  OutJob& o = out.j[0];
  o = OutJob{wide > 0 ? a.dxf : nb.c, nullptr, a.dx, a.in, 0, 0, {}, {}, {}};
  if (wide > 0 && nb.n > 0) {
    o.nbase = 2;
    o.stride = (long)a.T * a.in;
  }
  for (int p = 0; p < a.n_proj; ++p) {
    if (plan.slot_dl[p] < 0) continue;
    o.l[o.n_terms] = slot(a, plan.slot_dl[p]);
    o.v[o.n_terms] = a.p[p].a;
    o.s[o.n_terms] = a.p[p].scaling;
    ++o.n_terms;
  }
  return run_out<IO, true>(a, out, st);
}

}  // namespace

ProjScratchNeed proj_scratch_need(const ProjLaunch& a, bool backward) {
  ProjScratchNeed need{};
  bool narrow = false;
  for (int p = 0; p < a.n_proj; ++p) narrow = narrow || is_narrow(a, p);
  if (backward) {
    need.dxf = (long)a.T * a.in * (narrow ? 2 : 1);
  } else {
    const int splits = fwd_splits(a);
    for (int p = 0; p < a.n_proj; ++p)
      need.yf += (long)a.T * a.p[p].out * (is_narrow(a, p) ? splits : 1);
  }
  const RowsPlan plan = rows_plan(a, backward);
  if (plan.n > 0) {
    const long slabs = (a.T + 15) / 16, nt = (a.rank + 15) / 16;
    need.lowrank = (long)plan.n * a.T * a.rank;
    need.part = (long)plan.n * rows_splits(a, plan) * slabs * 256 * nt;
  }
  return need;
}

hipError_t launch_proj_forward(const ProjLaunch& a, hipStream_t st) {
  return a.io_bf16 ? forward_impl<bf16>(a, st) : forward_impl<float>(a, st);
}

hipError_t launch_proj_backward(const ProjLaunch& a, hipStream_t st) {
  return a.io_bf16 ? backward_impl<bf16>(a, st) : backward_impl<float>(a, st);
}

}  // namespace glacier
