// proj_gemm.hip -- the projection's narrow base products on the matrix
// cores (bf16 tensors): the k and v projections of a Qwen-style block have
// 512 outputs against 3584 inputs, a shape a library GEMM covers with a few
// dozen workgroups on a 256-CU chip.  Here every narrow projection of a call
// goes through one launch per direction, tiled finely enough to fill the
// chip:
//   forward   Yf_p[s] = X W_p^T over the s-th slice of the inputs   (NT)
//             64 outputs x 64 tokens per workgroup, the reduction split in
//             S slices; lowrank_out adds the S partials in slice order
//   backward  dXf2 = sum_p dY_p W_p over the narrow projections     (NN)
//             64 inputs x 64 tokens per workgroup, the projections'
//             reductions one after another; lowrank_out adds dXf2 to the
//             library GEMM's dXf
// GpuLoraEngine.ForwardQKV (GpuLoraEngine.Forward.cs:205-245) and
// LoraAdapter.Backward (LoraAdapter.cs:190-247) compute the same products.
//
// Both kernels compute the transposed tile C^T = (feature rows) x (token
// columns) with v_mfma_f32_16x16x32_bf16, so that a lane's four accumulators
// are four consecutive outputs of one token: one 16-byte store.  Stages of 64
// reduction elements go global -> registers -> LDS (rows of 144 bytes) with
// four stages' loads in flight while one is multiplied (a stage is only 8
// MFMAs per wave, far shorter than a load's round trip); one workgroup
// barrier per stage, the LDS double-buffered.  Loads go through buffer resources whose range
// ends at the last valid row, so rows past T or past a projection's outputs
// read as zero.  Fixed reduction order everywhere: bitwise repeatable.
#include "attn_common.hpp"
#include "proj_launch.hpp"

namespace glacier {
namespace {

constexpr int kGT = 64;       // tile rows (features) and columns (tokens)
constexpr int kGK = 64;       // reduction elements per stage
constexpr int kGS = kGK + 8;  // LDS row stride, elements (144 bytes)
constexpr int kGThreads = 256;
constexpr int kGTile = kGT * kGS;  // elements of one LDS operand tile
constexpr int kGPf = 4;            // stages in flight (registers) ahead of the one multiplied

// A row-major bf16 matrix seen from row `row0`: rows [row0, row0 + nrows)
// readable, anything past them zero.
struct RowSrc {
  __amdgpu_buffer_rsrc_t rs;
  int rowb;  // row stride in bytes
};

__device__ inline RowSrc row_src(const bf16* m, long ld, long row0, int nrows, int row_bytes) {
  const int rowb = static_cast<int>(ld * (long)sizeof(bf16));
  const int nrec = nrows <= 0 ? 0 : (nrows - 1) * rowb + row_bytes;
  const bf16* base = m + row0 * ld;
  const unsigned long long a = reinterpret_cast<unsigned long long>(base);
  const unsigned long long au =
      (static_cast<unsigned long long>(__builtin_amdgcn_readfirstlane(static_cast<int>(a >> 32))) << 32) |
      static_cast<unsigned>(__builtin_amdgcn_readfirstlane(static_cast<int>(a & 0xffffffffu)));
  RowSrc r;
  r.rs = __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void*>(au), (short)0,
                                           __builtin_amdgcn_readfirstlane(nrec), kBufferWord3);
  r.rowb = __builtin_amdgcn_readfirstlane(rowb);
  return r;
}

// One stage of one operand: 64 rows x 64 elements from column col0, two
// 16-byte pieces per thread (piece tid + 256 i: row / 8, 8-element column).
struct Stage {
  i32x4 w[2];
  __device__ inline void load(const RowSrc& s, int col0, int tid) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int idx = tid + kGThreads * i;
      const int off = (idx >> 3) * s.rowb + (col0 + 8 * (idx & 7)) * (int)sizeof(bf16);
      w[i] = __builtin_amdgcn_raw_buffer_load_b128(s.rs, off, 0, 0);
    }
  }
  __device__ inline void store(bf16* tile, int tid) const {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int idx = tid + kGThreads * i;
      *reinterpret_cast<i32x4*>(tile + (idx >> 3) * kGS + 8 * (idx & 7)) = w[i];
    }
  }
};

// The hardware deals workgroup ids to the 8 XCDs round-robin (id % 8), each
// XCD with its own L2.  Renumbering so that consecutive logical indices run
// on one XCD keeps the workgroups that share a weight tile (consecutive in
// both kernels' tile orders) on one L2: each XCD then fetches only its own
// share of the weights, instead of every XCD fetching all of them.
__device__ inline int xcd_logical(int id, int total) {
  constexpr int kXcds = 8;
  const int q = total / kXcds, r = total % kXcds, x = id % kXcds;
  return x * q + min(x, r) + id / kXcds;
}

__device__ inline f32x4 mfma_bf16(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// Lane (g, c) of wave (wf, wt) holds C^T rows f0 + 32 wf + 16 fb + 4g + r
// (features) of column t0 + 32 wt + 16 tb + c (token): C[token][f .. f + 3].
__device__ inline void store_tile(const f32x4 (&acc)[2][2], float* c, long ldc, int f0, int t0,
                                  int n_feat, int T, int wf, int wt, int lane) {
  const int g = lane >> 4, cl = lane & 15;
#pragma unroll
  for (int tb = 0; tb < 2; ++tb) {
    const int t = t0 + 32 * wt + 16 * tb + cl;
    if (t >= T) continue;
#pragma unroll
    for (int fb = 0; fb < 2; ++fb) {
      const int f = f0 + 32 * wf + 16 * fb + 4 * g;
      if (f < n_feat) *reinterpret_cast<f32x4*>(c + (long)t * ldc + f) = acc[fb][tb];
    }
  }
}

// ---------------------------------------------------------------------------
// Forward: workgroup b of job z is (split s, token tile, feature tile) with
// s fastest; the reduction covers inputs [s kchunk, (s + 1) kchunk) n K.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kGThreads) void proj_gemm_nt_kernel(const NarrowFwd a) {
  __shared__ __align__(16) bf16 lds[2][2][kGTile];  // [buffer][W, X]
  const int id = xcd_logical((int)blockIdx.x, (int)gridDim.x);
  int z = 0;
  while (z + 1 < a.n && id >= a.j[z + 1].first) ++z;
  const NarrowJob& job = a.j[z];
  const int b = id - job.first;
  const int s = b % a.nsplit, tile = b / a.nsplit;
  const int ttiles = (a.T + kGT - 1) / kGT;
  const int t0 = kGT * (tile % ttiles), f0 = kGT * (tile / ttiles);
  const int tid = threadIdx.x, lane = tid & 63, w = wave_id();
  const int wf = w & 1, wt = w >> 1, g = lane >> 4, c = lane & 15;
  const int k_begin = min(a.K, s * a.kchunk), k_end = min(a.K, k_begin + a.kchunk);
  const int nst = (k_end - k_begin) / kGK;
  const RowSrc ws = row_src(static_cast<const bf16*>(job.w), a.K, f0, job.n - f0, a.K * 2);
  const RowSrc xs = row_src(static_cast<const bf16*>(a.x), a.K, t0, a.T - t0, a.K * 2);

  f32x4 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  // kGPf stages in flight: stage st sits in register slot st % kGPf from
  // its load until it is stored to LDS buffer st % 2, kGPf stages later.
  // Every load is issued unconditionally (stages past the end read through a
  // zero-length resource, i.e. zeros, and add nothing), so the loop body has
  // no branch and the compiler waits only for the slot it stores.
  const RowSrc zero = row_src(static_cast<const bf16*>(job.w), a.K, 0, 0, 0);
  Stage pw[kGPf], px[kGPf];
  auto issue = [&](Stage& w_, Stage& x_, int st) {
    RowSrc w1 = zero, x1 = zero;
    if (st < nst) {
      w1 = ws;
      x1 = xs;
    }
    w_.load(w1, k_begin + kGK * st, tid);
    x_.load(x1, k_begin + kGK * st, tid);
  };
#pragma unroll
  for (int j = 0; j < kGPf; ++j) {
    issue(pw[j], px[j], j);
    __builtin_amdgcn_sched_barrier(0);  // slot order = issue order
  }
  for (int st0 = 0; st0 < nst; st0 += kGPf) {
#pragma unroll
    for (int j = 0; j < kGPf; ++j) {
      const int st = st0 + j;
      bf16* wl = lds[j & 1][0];
      bf16* xl = lds[j & 1][1];
      pw[j].store(wl, tid);
      px[j].store(xl, tid);
      __syncthreads();
      issue(pw[j], px[j], st + kGPf);
      // keep the loads of slot j here, before the products: scheduled later
      // they would be the newest loads when slot j is next stored, and that
      // store would wait for every load in flight
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int kk = 0; kk < kGK / 32; ++kk) {
        bf16x8 af[2], bf[2];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          af[i] = *reinterpret_cast<const bf16x8*>(wl + (32 * wf + 16 * i + c) * kGS + 32 * kk + 8 * g);
          bf[i] = *reinterpret_cast<const bf16x8*>(xl + (32 * wt + 16 * i + c) * kGS + 32 * kk + 8 * g);
        }
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int jj = 0; jj < 2; ++jj) acc[i][jj] = mfma_bf16(af[i], bf[jj], acc[i][jj]);
      }
    }
  }
  // partial s of this job: [T][n] at job.c + s T n (every split writes its
  // slice, zeros for an empty one, so the sum over slices is complete)
  store_tile(acc, job.c + (long)s * a.T * job.n, job.n, f0, t0, job.n, a.T, wf, wt, lane);
}

// ---------------------------------------------------------------------------
// Backward: workgroup (input tile, token tile); the reduction runs over the
// outputs of job 0, then job 1, ...  A operand W_p[k][f] read transposed from
// its row-major LDS tile (permuted k-slots {4g + r} U {16 + 4g + r} of each
// 32-step); B operand dY_p[t][k] read as the same slots, 8 bytes at a time.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kGThreads) void proj_gemm_nn_kernel(const NarrowBwd a) {
  __shared__ __align__(16) bf16 lds[2][2][kGTile];  // [buffer][W, dY]
  const int ttiles = (a.T + kGT - 1) / kGT;
  const int id = xcd_logical((int)blockIdx.x, (int)gridDim.x);
  const int t0 = kGT * (id % ttiles), f0 = kGT * (id / ttiles);
  const int tid = threadIdx.x, lane = tid & 63, w = wave_id();
  const int wf = w & 1, wt = w >> 1, g = lane >> 4, c = lane & 15;

  f32x4 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  // stage st belongs to job z with local reduction offset k0
  int nst = 0;
  for (int z = 0; z < a.n; ++z) nst += a.j[z].n / kGK;
  auto src = [&](int st, RowSrc& ws, RowSrc& ys, int& k0) {
    int z = 0, base = 0;
    while (z + 1 < a.n && st >= base + a.j[z].n / kGK) base += a.j[z++].n / kGK;
    const NarrowJob& job = a.j[z];
    k0 = kGK * (st - base);
    // W_p rows k0 .. k0 + 63 (of n), columns f0 ..; dY_p rows t0 .. (tokens)
    ws = row_src(static_cast<const bf16*>(job.w), a.K, k0, job.n - k0, a.K * 2);
    ys = row_src(static_cast<const bf16*>(job.dy), job.n, t0, a.T - t0, job.n * 2);
  };
  // as in the forward: loads unconditional, stages past the end zeros
  const RowSrc zero = row_src(static_cast<const bf16*>(a.j[0].w), a.K, 0, 0, 0);
  Stage pw[kGPf], py[kGPf];
  auto issue = [&](Stage& w_, Stage& y_, int st) {
    RowSrc ws = zero, ys = zero;
    int k0 = 0;
    if (st < nst) src(st, ws, ys, k0);
    w_.load(ws, f0, tid);
    y_.load(ys, k0, tid);
  };
#pragma unroll
  for (int j = 0; j < kGPf; ++j) {
    issue(pw[j], py[j], j);
    __builtin_amdgcn_sched_barrier(0);
  }
  for (int st0 = 0; st0 < nst; st0 += kGPf) {
#pragma unroll
    for (int j = 0; j < kGPf; ++j) {
      const int st = st0 + j;
      bf16* wl = lds[j & 1][0];  // [k][f]
      bf16* yl = lds[j & 1][1];  // [t][k]
      pw[j].store(wl, tid);
      py[j].store(yl, tid);
      __syncthreads();
      issue(pw[j], py[j], st + kGPf);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int kk = 0; kk < kGK / 32; ++kk) {
        bf16x8 af[2], bf[2];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          const bf16x4 lo = read_tr<kGS>(wl, 32 * kk, 32 * wf + 16 * i, lane);
          const bf16x4 hi = read_tr<kGS>(wl, 32 * kk + 16, 32 * wf + 16 * i, lane);
          const bf16* yr = yl + (32 * wt + 16 * i + c) * kGS + 32 * kk + 4 * g;
          const bf16x4 ylo = *reinterpret_cast<const bf16x4*>(yr);
          const bf16x4 yhi = *reinterpret_cast<const bf16x4*>(yr + 16);
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            af[i][r] = lo[r];
            af[i][4 + r] = hi[r];
            bf[i][r] = ylo[r];
            bf[i][4 + r] = yhi[r];
          }
        }
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int jj = 0; jj < 2; ++jj) acc[i][jj] = mfma_bf16(af[i], bf[jj], acc[i][jj]);
      }
    }
  }
  store_tile(acc, a.c, a.K, f0, t0, a.K, a.T, wf, wt, lane);
}

}  // namespace

bool narrow_gemm_fits(int in_features, int out_features) {
  return in_features % kGK == 0 && out_features % kGK == 0 && out_features <= kNarrowMaxOut;
}

int narrow_fwd_splits(int T, int total_feature_tiles) {
  const int tiles = ((T + kGT - 1) / kGT) * total_feature_tiles;
  int s = 1;
  while (s < 4 && tiles * s * 2 <= 256) s *= 2;  // at least one workgroup per CU if it takes <= 4
  return s;
}

int narrow_feature_tiles(int out_features) { return (out_features + kGT - 1) / kGT; }

hipError_t launch_narrow_fwd(NarrowFwd a, hipStream_t st) {
  const int ttiles = (a.T + kGT - 1) / kGT;
  int total = 0;
  for (int z = 0; z < a.n; ++z) {
    a.j[z].first = total;
    total += ttiles * narrow_feature_tiles(a.j[z].n) * a.nsplit;
  }
  if (total == 0) return hipSuccess;
  hipLaunchKernelGGL(proj_gemm_nt_kernel, dim3(total), dim3(kGThreads), 0, st, a);
  return hipGetLastError();
}

hipError_t launch_narrow_bwd(const NarrowBwd& a, hipStream_t st) {
  const int ttiles = (a.T + kGT - 1) / kGT, ftiles = (a.K + kGT - 1) / kGT;
  if (ttiles == 0 || ftiles == 0) return hipSuccess;
  hipLaunchKernelGGL(proj_gemm_nn_kernel, dim3(ttiles * ftiles), dim3(kGThreads), 0, st, a);
  return hipGetLastError();
}

}  // namespace glacier
