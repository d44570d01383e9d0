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
#include "lds_mfma.hpp"
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

// ---------------------------------------------------------------------------
// Wide projections (bf16 tensors; q of a Qwen-style block: 3584 x 3584): a
// workgroup computes a 128-feature x 64-token tile of C^T on
// v_mfma_f32_32x32x16_bf16, 4 waves of 64 features x 32 tokens each (two
// 32 x 32 accumulator blocks per wave).  Stages of 64 reduction elements go
// global -> LDS by DMA (buffer_load ... lds, 16 bytes a lane) into a 4-slot
// ring, three stages ahead; one workgroup barrier per stage.  Rows are
// unpadded with their 16-byte pieces XOR-swizzled (lds_sw), so the fragment
// reads (16 rows x one piece per quarter-wave) and the transposing reads of
// the backward (4 rows x 4 pieces per half-wave) are free of bank conflicts.
//   forward  (NT) C^T[f][t] = sum_k W[f][k] X[t][k]: both operands are read
//            as fragments, A from the [128][64] W tile, B from the [64][64]
//            X tile;
//   backward (NN) C^T[c][t] = sum_f W[f][c] dY[t][f]: A from the [64 f][128 c]
//            W tile by ds_read_b64_tr_b16 (four f of one column per read,
//            two reads per k-step), B from the [64][64] dY tile.
// MFMA layout (lane l, c = l % 32, h = l / 32): A[row c][k = 8h .. 8h + 7],
// B[k = 8h ..][col c]; accumulator element e holds column c, row
// 8 (e / 4) + 4h + e % 4, so each group of four is four consecutive
// features of one token: one 16-byte store.
// ---------------------------------------------------------------------------
constexpr int kWF = 128;                 // features per tile
constexpr int kWT = 64;                  // tokens per tile
constexpr int kWK = 64;                  // reduction elements per stage
constexpr int kWA = kWF * kWK * 2;       // A tile bytes (16 KB)
constexpr int kWB = kWT * kWK * 2;       // B tile bytes (8 KB)
constexpr int kWStage = kWA + kWB;       // one ring slot
constexpr int kWRing = 4;
constexpr int kWThreads = 256;
constexpr int kWDma = (kWA + kWB) / 1024 / 4;  // DMA instructions per wave per stage (6)

static_assert(kWRing * kWStage <= 160 * 1024, "ring exceeds the LDS of a CU");
static_assert(kWStage + 4096 * 3 < 65536, "read immediates fit their 16-bit field");

#if defined(__HIP_DEVICE_COMPILE__)
__device__ inline f32x16 mma32(const bf16x8& a, const bf16x8& b, const f32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// Per-lane DMA offsets of 128-byte rows (8 pieces): instruction n covers
// rows 8 n .. 8 n + 7; lane l writes slot l % 8 of row 8 n + l / 8 and
// fetches the global piece slot ^ lds_sw<64>(row), which repeats every two
// instructions.  256-byte rows (16 pieces): rows 4 n .. 4 n + 3, slot l % 16,
// piece slot ^ lds_sw<128>(row), repeating every four instructions.
__device__ inline int dma_off128(int lane, int n, int rowb) {
  const int r = 8 * n + (lane >> 3), slot = lane & 7;
  return (lane >> 3) * rowb + 16 * (slot ^ lds_sw<64>(r));
}
__device__ inline int dma_off256(int lane, int n, int rowb) {
  const int r = 4 * n + (lane >> 4), slot = lane & 15;
  return (lane >> 4) * rowb + 16 * (slot ^ lds_sw<128>(r));
}

// Byte offset, inside a tile of 128-byte rows, of this lane's fragment read
// of k-step 0 for rows row0 + lane % 32 (row0 a multiple of 16); k-step s
// reads at that offset ^ 32 s.
__device__ inline unsigned frag_off128(int lane, int row0) {
  const int r = row0 + (lane & 31), h = lane >> 5;
  return static_cast<unsigned>(r * 128 + 16 * (h ^ lds_sw<64>(r)));
}
// Byte offset, inside a tile of 256-byte rows, of this lane's transposing
// read j (0, 1) of k-step 0 for columns col0 + 16 (G & 1) + 4 (i & 3)
// (quarter-wave G, lane i in it): rows 8 h + 4 j + i / 4; k-step s reads
// 16 s rows further (+4096 s), the 32 columns after col0 at ^ 64.
__device__ inline unsigned tr_off256(int lane, int col0, int j) {
  const int G = lane >> 4, i = lane & 15, h = lane >> 5;
  const int r = 8 * h + 4 * j + (i >> 2);
  const int col = col0 + 16 * (G & 1) + 4 * (i & 3);
  return static_cast<unsigned>(r * 256 + 16 * ((col >> 3) ^ lds_sw<128>(r)) + 2 * (col & 7));
}

// Stores this wave's two 32 x 32 blocks (features fw + 32 fb, tokens tw) of
// C^T into C [T][ldc] (fp32), rows past T skipped.
__device__ inline void store_wide(const f32x16 (&acc)[2], float* c, long ldc, int fw, int tw, int T,
                                  int lane) {
  const int t = tw + (lane & 31), h = lane >> 5;
  if (t >= T) return;
#pragma unroll
  for (int fb = 0; fb < 2; ++fb)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int f = fw + 32 * fb + 8 * q + 4 * h;
      *reinterpret_cast<f32x4*>(c + (long)t * ldc + f) =
          f32x4{acc[fb][4 * q], acc[fb][4 * q + 1], acc[fb][4 * q + 2], acc[fb][4 * q + 3]};
    }
}
#endif

// The stage loop shared by both directions: prologue of three stages, then
// per stage: wait for this wave's DMA of the stage (the two later stages
// stay in flight), barrier, DMA of the stage three ahead into the slot just
// freed (every wave's reads of it completed before the barrier) (unconditional: past the end
// it reads through an empty resource), then the stage's products.  The ring
// slot of every read is an immediate offset: slots 0, 1 from the lane's
// addresses as given, slots 2, 3 from the same + 2 kWStage.
template <typename Issue, typename Compute>
__device__ inline void wide_loop(int nst, Issue&& issue, Compute&& compute) {
  issue(0, 0);
  issue(1, 1);
  issue(2, 2);
  int st = 0;
  auto one = [&](auto slot) {
    constexpr int SL = decltype(slot)::value;
    vmw<2 * kWDma>();
    wg_barrier();
    issue(st + 3, (SL + 3) & 3);
    compute(slot);
    ++st;
  };
#pragma clang loop unroll(disable)
  while (st + 3 < nst) {
    one(std::integral_constant<int, 0>{});
    one(std::integral_constant<int, 1>{});
    one(std::integral_constant<int, 2>{});
    one(std::integral_constant<int, 3>{});
  }
  if (st < nst) one(std::integral_constant<int, 0>{});
  if (st < nst) one(std::integral_constant<int, 1>{});
  if (st < nst) one(std::integral_constant<int, 2>{});
  vmw<0>();  // the DMA issued past the end lands before the workgroup ends
}

__global__ __launch_bounds__(kWThreads) void proj_gemm_wide_nt_kernel(const WideFwd a) {
#if defined(__HIP_DEVICE_COMPILE__)
  __shared__ __align__(1024) unsigned char lds[kWRing * kWStage];
  const int ttiles = (a.T + kWT - 1) / kWT;
  const int id = xcd_logical((int)blockIdx.x, (int)gridDim.x);
  const int t0 = kWT * (id % ttiles), f0 = kWF * (id / ttiles);
  const int lane = threadIdx.x & 63, w = wave_id();
  const int wf = w & 1, wt = w >> 1;
  const int rowb = a.K * 2;
  // A: W rows f0 .., B: X rows t0 .. (rows past T read as zeros)
  const __amdgpu_buffer_rsrc_t ra =
      wave_rsrc(static_cast<const bf16*>(a.w) + (long)f0 * a.K, kWF * rowb);
  const __amdgpu_buffer_rsrc_t rb = wave_rsrc(static_cast<const bf16*>(a.x) + (long)t0 * a.K,
                                              max(0, min(kWT, a.T - t0)) * rowb);
  const __amdgpu_buffer_rsrc_t rz = wave_rsrc(a.x, 0);
  // this wave's DMA: A rows 32 w .. 32 w + 31 (4 instructions; every row
  // valid, the row block in the scalar offset), B rows 16 w .. 16 w + 15 (2
  // instructions; the row in the per-lane offset, which alone is checked
  // against the resource's range, so rows past T read as zeros)
  const int oa0 = dma_off128(lane, 0, rowb), oa1 = dma_off128(lane, 1, rowb);
  const int ob0 = dma_off128(lane, 0, rowb) + 16 * w * rowb, ob1 = dma_off128(lane, 1, rowb) + (16 * w + 8) * rowb;
  const unsigned sbase = static_cast<unsigned>(reinterpret_cast<uintptr_t>((GLACIER_LDS void*)lds));
  auto issue = [&](int st, int slot) {
    const bool live = st < a.K / kWK;
    const __amdgpu_buffer_rsrc_t sa = live ? ra : rz, sb = live ? rb : rz;
    unsigned char* base = lds + slot * kWStage;
    const int k0 = st * kWK * 2;
#pragma unroll
    for (int n = 0; n < 4; ++n)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(sa, (GLACIER_LDS void*)(base + (32 * w + 8 * n) * 128), 16,
                                               (n & 1) ? oa1 : oa0, (32 * w + 8 * n) * rowb + k0, 0, 0);
#pragma unroll
    for (int n = 0; n < 2; ++n)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(sb, (GLACIER_LDS void*)(base + kWA + (16 * w + 8 * n) * 128),
                                               16, n ? ob1 : ob0, k0, 0, 0);
  };
  // read addresses: A rows 64 wf + 32 fb (fb at +4096), B rows 32 wt; k-step s
  unsigned fa[2][4], fbb[2][4];
  {
    const unsigned oa = frag_off128(lane, 64 * wf), ob = frag_off128(lane, 32 * wt);
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      fa[0][s] = sbase + (oa ^ (32u * s));
      fbb[0][s] = sbase + kWA + (ob ^ (32u * s));
      fa[1][s] = fa[0][s] + 2 * kWStage;
      fbb[1][s] = fbb[0][s] + 2 * kWStage;
    }
  }
  f32x16 acc[2];
#pragma unroll
  for (int fb = 0; fb < 2; ++fb)
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[fb][e] = 0.0f;
  auto compute = [&](auto slot) {
    constexpr int SL = decltype(slot)::value, HS = SL >> 1, OFF = (SL & 1) * kWStage;
    bf16x8 ra_[4][2], rb_[4];
    auto rd = [&](auto sc) {
      constexpr int S = decltype(sc)::value;
      ra_[S][0] = rd128<OFF>(fa[HS][S]);
      ra_[S][1] = rd128<OFF + 4096>(fa[HS][S]);
      rb_[S] = rd128<OFF>(fbb[HS][S]);
    };
    rd(std::integral_constant<int, 0>{});
    rd(std::integral_constant<int, 1>{});
    static_for<4>([&](auto sc) {
      constexpr int S = decltype(sc)::value;
      if constexpr (S + 2 < 4) {
        lgkm<3>();
        rd(std::integral_constant<int, S + 2>{});
        lgkm<6>();
      } else if constexpr (S == 2) {
        lgkm<3>();
      } else {
        lgkm<0>();
      }
      tie_v(ra_[S][0]);
      tie_v(ra_[S][1]);
      tie_v(rb_[S]);
      acc[0] = mma32(ra_[S][0], rb_[S], acc[0]);
      acc[1] = mma32(ra_[S][1], rb_[S], acc[1]);
    });
  };
  wide_loop(a.K / kWK, issue, compute);
  store_wide(acc, a.c, a.n, f0 + 64 * wf, t0 + 32 * wt, a.T, lane);
#endif
}

__global__ __launch_bounds__(kWThreads) void proj_gemm_wide_nn_kernel(const WideBwd a) {
#if defined(__HIP_DEVICE_COMPILE__)
  __shared__ __align__(1024) unsigned char lds[kWRing * kWStage];
  const int ttiles = (a.T + kWT - 1) / kWT;
  const int id = xcd_logical((int)blockIdx.x, (int)gridDim.x);
  const int t0 = kWT * (id % ttiles), c0 = kWF * (id / ttiles);
  const int lane = threadIdx.x & 63, w = wave_id();
  const int wf = w & 1, wt = w >> 1;
  const int rowbw = a.K * 2;
  int nst = 0;
  for (int z = 0; z < a.n; ++z) nst += a.j[z].n / kWK;
  const __amdgpu_buffer_rsrc_t rz = wave_rsrc(a.j[0].w, 0);
  const int ow[4] = {dma_off256(lane, 0, rowbw), dma_off256(lane, 1, rowbw), dma_off256(lane, 2, rowbw),
                     dma_off256(lane, 3, rowbw)};
  const unsigned sbase = static_cast<unsigned>(reinterpret_cast<uintptr_t>((GLACIER_LDS void*)lds));
  // the job of the stages being issued (stages are issued in order): its
  // resources over W_z (from column c0) and dY_z (from token t0), its first
  // stage and the first stage of the next job
  int z = -1, zbase = 0, zend = 0, rowby = 0, oy0 = 0, oy1 = 0;
  __amdgpu_buffer_rsrc_t ra = rz, rb = rz;
  auto issue = [&](int st, int slot) {
    while (st >= zend && z + 1 < a.n) {
      ++z;
      zbase = zend;
      zend += a.j[z].n / kWK;
      const WideJob& job = a.j[z];
      rowby = job.n * 2;
      ra = wave_rsrc(static_cast<const bf16*>(job.w) + c0, (job.n - 1) * rowbw + kWF * 2);
      rb = wave_rsrc(static_cast<const bf16*>(job.dy) + (long)t0 * job.n,
                     max(0, min(kWT, a.T - t0)) * rowby);
      // the row in the per-lane offset (checked against the range: rows
      // past T read as zeros), the column f0 in the scalar one
      oy0 = dma_off128(lane, 0, rowby) + 16 * w * rowby;
      oy1 = dma_off128(lane, 1, rowby) + (16 * w + 8) * rowby;
    }
    const bool live = st < nst;
    const __amdgpu_buffer_rsrc_t sa = live ? ra : rz, sb = live ? rb : rz;
    const int f0 = (st - zbase) * kWK;  // the job's reduction rows f0 .. f0 + 63
    unsigned char* base = lds + slot * kWStage;
    // A: W_z[f0 + r][c0 ..] (256-byte rows); B: dY_z[t0 + r][f0 ..] (128 bytes)
#pragma unroll
    for (int n = 0; n < 4; ++n)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(sa, (GLACIER_LDS void*)(base + (16 * w + 4 * n) * 256), 16,
                                               ow[n], (f0 + 16 * w + 4 * n) * rowbw, 0, 0);
#pragma unroll
    for (int n = 0; n < 2; ++n)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(sb, (GLACIER_LDS void*)(base + kWA + (16 * w + 8 * n) * 128),
                                               16, n ? oy1 : oy0, 2 * f0, 0, 0);
  };
  // read addresses: A transposed, columns 64 wf + 32 fb (fb: ^ 64), reads j;
  // B fragments rows 32 wt, k-step s
  unsigned ta[2][2][2], fbb[2][4];
  {
    const unsigned o0 = tr_off256(lane, 64 * wf, 0), o1 = tr_off256(lane, 64 * wf, 1);
    const unsigned ob = frag_off128(lane, 32 * wt);
#pragma unroll
    for (int hs = 0; hs < 2; ++hs) {
#pragma unroll
      for (int fb = 0; fb < 2; ++fb) {
        ta[hs][fb][0] = sbase + 2u * kWStage * hs + (o0 ^ (64u * fb));
        ta[hs][fb][1] = sbase + 2u * kWStage * hs + (o1 ^ (64u * fb));
      }
#pragma unroll
      for (int s = 0; s < 4; ++s) fbb[hs][s] = sbase + 2u * kWStage * hs + kWA + (ob ^ (32u * s));
    }
  }
  f32x16 acc[2];
#pragma unroll
  for (int fb = 0; fb < 2; ++fb)
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[fb][e] = 0.0f;
  auto compute = [&](auto slot) {
    constexpr int SL = decltype(slot)::value, HS = SL >> 1, OFF = (SL & 1) * kWStage;
    bf16x4 rt[4][2][2];
    bf16x8 rb_[4];
    auto rd = [&](auto sc) {
      constexpr int S = decltype(sc)::value;
#pragma unroll
      for (int fb = 0; fb < 2; ++fb) {
        rt[S][fb][0] = rdtr<OFF + 4096 * S>(ta[HS][fb][0]);
        rt[S][fb][1] = rdtr<OFF + 4096 * S>(ta[HS][fb][1]);
      }
      rb_[S] = rd128<OFF>(fbb[HS][S]);
    };
    rd(std::integral_constant<int, 0>{});
    rd(std::integral_constant<int, 1>{});
    static_for<4>([&](auto sc) {
      constexpr int S = decltype(sc)::value;
      if constexpr (S + 2 < 4) {
        lgkm<5>();
        rd(std::integral_constant<int, S + 2>{});
        lgkm<10>();
      } else if constexpr (S == 2) {
        lgkm<5>();
      } else {
        lgkm<0>();
      }
#pragma unroll
      for (int fb = 0; fb < 2; ++fb) {
        tie_v(rt[S][fb][0]);
        tie_v(rt[S][fb][1]);
      }
      tie_v(rb_[S]);
      acc[0] = mma32(join8(rt[S][0][0], rt[S][0][1]), rb_[S], acc[0]);
      acc[1] = mma32(join8(rt[S][1][0], rt[S][1][1]), rb_[S], acc[1]);
    });
  };
  wide_loop(nst, issue, compute);
  store_wide(acc, a.c, a.K, c0 + 64 * wf, t0 + 32 * wt, a.T, lane);
#endif
}

// ---------------------------------------------------------------------------
// Every other projection (fp32 tensors, the fp32-operand mode, or bf16
// tensors of a shape neither kernel above takes): both directions on
// v_mfma_f32_16x16x4f32, any shape, operands converted to fp32 on load.  A workgroup computes a 64-feature x
// 64-token tile of C^T, 4 waves of 32 x 32 (2 x 2 blocks of 16 x 16).
// Stages of 32 reduction elements go global -> registers -> LDS (two
// buffers, one barrier per stage, the next stage's loads in flight during
// the products); elements past any edge load as zero.
//   forward  (NT) C^T[f][t] = sum_k W[f][k] X[t][k]   (A tile [f][k])
//   backward (NN) C^T[c][t] = sum_z sum_f W_z[f][c] dY_z[t][f]   (A tile [f][c])
// MFMA layout (lane l, c = l % 16, g = l / 16): A[row c][k = g],
// B[k = g][col c]; accumulator i holds column c, row 4 g + i: four
// consecutive features of one token.
// ---------------------------------------------------------------------------
constexpr int kFT = 64;       // features and tokens per tile
constexpr int kFK = 32;       // reduction elements per stage
constexpr int kFS = kFK + 4;  // row stride of [row][k] tiles (floats): conflict-free
constexpr int kFC = kFT + 16; // row stride of the backward's [k][feature] tile
constexpr int kFThreads = 256;

// Four elements k .. k + 3 of a row (len elements valid) as fp32, zero past
// the end; vec: the row allows one aligned vector load.
template <typename IO>
__device__ inline f32x4 load4_f32(const IO* row, int k, int len, bool vec) {
  if (vec && k + 3 < len) {
    if constexpr (sizeof(IO) == 4) {
      return *reinterpret_cast<const f32x4*>(row + k);
    } else {
      const bf16x4 h = *reinterpret_cast<const bf16x4*>(row + k);
      return f32x4{(float)h[0], (float)h[1], (float)h[2], (float)h[3]};
    }
  }
  f32x4 v;
#pragma unroll
  for (int i = 0; i < 4; ++i) v[i] = k + i < len ? (float)row[k + i] : 0.0f;
  return v;
}

template <typename IO, bool NN>
__global__ __launch_bounds__(kFThreads) void proj_gemm_f32_kernel(const WideFwd fa, const WideBwd ba) {
  __shared__ __align__(16) float la[2][NN ? kFK * kFC : kFT * kFS];
  __shared__ __align__(16) float lb[2][kFT * kFS];
  const int T = NN ? ba.T : fa.T;
  const int nout = NN ? ba.K : fa.n;  // C^T rows: features
  const int ttiles = (T + kFT - 1) / kFT;
  const int id = xcd_logical((int)blockIdx.x, (int)gridDim.x);
  const int t0 = kFT * (id % ttiles), f0 = kFT * (id / ttiles);
  const int tid = threadIdx.x, lane = tid & 63, w = wave_id();
  const int wf = w & 1, wt = w >> 1, c = lane & 15, g = lane >> 4;
  // stages: forward over K; backward over every job's outputs in turn
  int nst = 0;
  if constexpr (NN) {
    for (int z = 0; z < ba.n; ++z) nst += (ba.j[z].n + kFK - 1) / kFK;
  } else {
    nst = (fa.K + kFK - 1) / kFK;
  }
  f32x4 ra[2], rb[2];
  auto load = [&](int st) {
    const IO* wsrc;
    const IO* bsrc;
    int k0, klen, bstride;
    if constexpr (NN) {
      int z = 0, base = 0;
      while (z + 1 < ba.n && st >= base + (ba.j[z].n + kFK - 1) / kFK) base += (ba.j[z++].n + kFK - 1) / kFK;
      k0 = kFK * (st - base);
      klen = ba.j[z].n;
      wsrc = static_cast<const IO*>(ba.j[z].w);
      bsrc = static_cast<const IO*>(ba.j[z].dy);
      bstride = klen;
    } else {
      k0 = kFK * st;
      klen = fa.K;
      wsrc = static_cast<const IO*>(fa.w);
      bsrc = static_cast<const IO*>(fa.x);
      bstride = fa.K;
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int idx = tid + kFThreads * i;
      if constexpr (NN) {
        // A: W_z rows k0 + idx / 16 (of klen), columns f0 + 4 (idx % 16)
        const int kr = k0 + (idx >> 4), cc = f0 + 4 * (idx & 15);
        ra[i] = kr < klen ? load4_f32(wsrc + (long)kr * ba.K, cc, nout, (ba.K & 3) == 0) : f32x4{0, 0, 0, 0};
      } else {
        // A: W rows f0 + idx / 8, columns k0 + 4 (idx % 8)
        const int fr = f0 + (idx >> 3), kc = k0 + 4 * (idx & 7);
        ra[i] = fr < nout ? load4_f32(wsrc + (long)fr * fa.K, kc, klen, (fa.K & 3) == 0) : f32x4{0, 0, 0, 0};
      }
      // B: rows t0 + idx / 8 (tokens), columns k0 + 4 (idx % 8)
      const int tr = t0 + (idx >> 3), kc = k0 + 4 * (idx & 7);
      rb[i] = tr < T ? load4_f32(bsrc + (long)tr * bstride, kc, klen, (bstride & 3) == 0) : f32x4{0, 0, 0, 0};
    }
  };
  auto store = [&](int buf) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int idx = tid + kFThreads * i;
      if constexpr (NN)
        *reinterpret_cast<f32x4*>(&la[buf][(idx >> 4) * kFC + 4 * (idx & 15)]) = ra[i];
      else
#pragma unroll
        for (int e = 0; e < 4; ++e) la[buf][(idx >> 3) * kFS + 4 * (idx & 7) + e] = ra[i][e];
#pragma unroll
      for (int e = 0; e < 4; ++e) lb[buf][(idx >> 3) * kFS + 4 * (idx & 7) + e] = rb[i][e];
    }
  };
  f32x4 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  if (nst > 0) {
    load(0);
    store(0);
  }
  __syncthreads();
  for (int st = 0; st < nst; ++st) {
    const int buf = st & 1;
    if (st + 1 < nst) load(st + 1);
#pragma unroll
    for (int kk = 0; kk < kFK / 4; ++kk) {
      float av[2], bv[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int fr = 32 * wf + 16 * i + c, tr = 32 * wt + 16 * i + c, k = 4 * kk + g;
        av[i] = NN ? la[buf][k * kFC + fr] : la[buf][fr * kFS + k];
        bv[i] = lb[buf][tr * kFS + k];
      }
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[i], bv[j], acc[i][j], 0, 0, 0);
    }
    if (st + 1 < nst) store(buf ^ 1);
    __syncthreads();
  }
  // C [T][nout]: token t0 + 32 wt + 16 j + c, features f0 + 32 wf + 16 i + 4 g ..
  float* cdst = NN ? ba.c : fa.c;
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int t = t0 + 32 * wt + 16 * j + c;
    if (t >= T) continue;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int f = f0 + 32 * wf + 16 * i + 4 * g;
      float* d = cdst + (long)t * nout + f;
      // backward after the wide kernel: add to what it wrote
      const bool add = NN && ba.accumulate;
      if (f + 3 < nout && (nout & 3) == 0) {
        f32x4 v = acc[i][j];
        if (add) v += *reinterpret_cast<const f32x4*>(d);
        *reinterpret_cast<f32x4*>(d) = v;
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (f + e < nout) d[e] = add ? d[e] + acc[i][j][e] : acc[i][j][e];
      }
    }
  }
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

bool wide_gemm_fits(int in_features, int out_features) {
  return in_features % kWF == 0 && out_features % kWF == 0;
}

hipError_t launch_wide_fwd(const WideFwd& a, hipStream_t st) {
  const int ttiles = (a.T + kWT - 1) / kWT, ftiles = a.n / kWF;
  if (ttiles == 0 || ftiles == 0) return hipSuccess;
  if (a.K % kWK != 0 || a.n % kWF != 0) return hipErrorInvalidValue;
  hipLaunchKernelGGL(proj_gemm_wide_nt_kernel, dim3(ttiles * ftiles), dim3(kWThreads), 0, st, a);
  return hipGetLastError();
}

hipError_t launch_wide_bwd(const WideBwd& a, hipStream_t st) {
  const int ttiles = (a.T + kWT - 1) / kWT, ftiles = a.K / kWF;
  if (ttiles == 0 || ftiles == 0 || a.n == 0) return hipSuccess;
  if (a.K % kWF != 0) return hipErrorInvalidValue;
  for (int z = 0; z < a.n; ++z)
    if (a.j[z].n % kWK != 0) return hipErrorInvalidValue;
  hipLaunchKernelGGL(proj_gemm_wide_nn_kernel, dim3(ttiles * ftiles), dim3(kWThreads), 0, st, a);
  return hipGetLastError();
}

hipError_t launch_generic_fwd(const WideFwd& a, bool io_bf16, hipStream_t st) {
  const int ttiles = (a.T + kFT - 1) / kFT, ftiles = (a.n + kFT - 1) / kFT;
  if (ttiles == 0 || ftiles == 0) return hipSuccess;
  auto fn = io_bf16 ? proj_gemm_f32_kernel<bf16, false> : proj_gemm_f32_kernel<float, false>;
  hipLaunchKernelGGL(fn, dim3(ttiles * ftiles), dim3(kFThreads), 0, st, a, WideBwd{});
  return hipGetLastError();
}

hipError_t launch_generic_bwd(const WideBwd& a, bool io_bf16, hipStream_t st) {
  const int ttiles = (a.T + kFT - 1) / kFT, ftiles = (a.K + kFT - 1) / kFT;
  if (ttiles == 0 || ftiles == 0 || a.n == 0) return hipSuccess;
  auto fn = io_bf16 ? proj_gemm_f32_kernel<bf16, true> : proj_gemm_f32_kernel<float, true>;
  hipLaunchKernelGGL(fn, dim3(ttiles * ftiles), dim3(kFThreads), 0, st, WideFwd{}, a);
  return hipGetLastError();
}

hipError_t launch_narrow_bwd(const NarrowBwd& a, hipStream_t st) {
  const int ttiles = (a.T + kGT - 1) / kGT, ftiles = (a.K + kGT - 1) / kGT;
  if (ttiles == 0 || ftiles == 0) return hipSuccess;
  hipLaunchKernelGGL(proj_gemm_nn_kernel, dim3(ttiles * ftiles), dim3(kGThreads), 0, st, a);
  return hipGetLastError();
}

}  // namespace glacier
