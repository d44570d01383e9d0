// attn_launch.hpp -- host-side interface between the engine and the kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include <algorithm>
#include <type_traits>
#include <utility>
#include <vector>

namespace glacier {

constexpr int kTile = 64;      // queries or keys per workgroup tile
constexpr int kWideTile = 128; // rows per tile of the 32x32x16-MFMA backward
constexpr int kWaves = 4;      // waves per workgroup, 16 rows each
constexpr int kThreads = 256;  // kWaves * 64
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.69314718055994531f;
constexpr float kNegBig = -1.0e30f;  // running-max start value (finite)

// One 64-row tile of one packed sequence.
struct TileDesc {
  int32_t tok0;   // first token of the sequence in the [T][H][D] tensors
  int32_t len;    // tokens in the sequence
  int32_t tile;   // tile index inside the sequence (rows 64*tile ..)
  int32_t kind;   // backward table: a TileKind (unused elsewhere)
};

// Backward tile kinds.  A split dK/dV tile runs as two workgroups, each over
// half of the tile's query tiles (the first half holds the diagonal one); the
// second half writes its own partials, which the head reduction adds.
enum TileKind : int {
  kTileDkDv = 0,
  kTileDq = 1,
  kTileDkDvFirstHalf = 2,
  kTileDkDvSecondHalf = 3,
  kTileDqSecond = 4,  // wide backward over head pairs: the dQ tile of the pair's second head
};
// dK/dV tiles 0 .. split - 1 of each sequence may be split (16-row backward,
// bf16 tensors, only while the launch about fits one workgroup per CU).
constexpr int kBwdMaxSplit = 3;

constexpr int kPrecFp32 = 0;
constexpr int kPrecBf16 = 1;

// Kernel kinds, in launch order.
enum KernelId : int {
  kKernRopeK = 0,
  kKernFwd = 1,
  kKernBwd = 2,
  kKernReduce = 3,
  kKernNormFwd = 4,  // rmsnorm.hip
  kKernNormBwd = 5,
  kKernBwdStats = 6,  // attn_bwd.hip: row stats before the bf16 backward
  kKernCount = 7,
};

// Optional per-kernel hipEvent timing on the launch stream.
class KernelTimer {
 public:
  bool enabled = false;
  ~KernelTimer() { reset(); }
  void reset() {
    for (auto& p : pending_) {
      (void)hipEventDestroy(p.second.first);
      (void)hipEventDestroy(p.second.second);
    }
    pending_.clear();
    for (int i = 0; i < kKernCount; ++i) {
      total_ms_[i] = 0.0;
      launches_[i] = 0;
    }
  }
  void record(int id, hipEvent_t a, hipEvent_t b) { pending_.push_back({id, {a, b}}); }
  // Folds finished event pairs into the totals (call after a synchronize).
  hipError_t collect() {
    for (auto& p : pending_) {
      float ms = 0.0f;
      hipError_t e = hipEventElapsedTime(&ms, p.second.first, p.second.second);
      if (e != hipSuccess) return e;
      total_ms_[p.first] += ms;
      launches_[p.first] += 1;
      (void)hipEventDestroy(p.second.first);
      (void)hipEventDestroy(p.second.second);
    }
    pending_.clear();
    return hipSuccess;
  }
  double total_ms(int id) const { return total_ms_[id]; }
  int64_t launches(int id) const { return launches_[id]; }

 private:
  std::vector<std::pair<int, std::pair<hipEvent_t, hipEvent_t>>> pending_;
  double total_ms_[kKernCount] = {};
  int64_t launches_[kKernCount] = {};
};

// Event pair for one timed launch.  The launch itself timestamps the events
// (hipExtLaunchKernelGGL writes them from the kernel's dispatch packet), so
// the interval is the kernel's own execution and no extra packets enter the
// stream.  With timing off both events are null and the launch is a plain one.
class LaunchTiming {
 public:
  LaunchTiming(KernelTimer* tm, int id) : tm_(tm), id_(id) {
    if (tm_ != nullptr && tm_->enabled) {
      if (hipEventCreate(&a_) == hipSuccess && hipEventCreate(&b_) == hipSuccess) {
        on_ = true;
      } else {
        release();
      }
    }
  }
  hipEvent_t start() const { return a_; }
  hipEvent_t stop() const { return b_; }
  // Call after a successful launch: the pair joins the timer's pending list.
  void launched() {
    if (on_) tm_->record(id_, a_, b_);
    on_ = false;
    a_ = b_ = nullptr;
  }
  ~LaunchTiming() { release(); }

 private:
  void release() {
    if (a_ != nullptr) (void)hipEventDestroy(a_);
    if (b_ != nullptr) (void)hipEventDestroy(b_);
    a_ = b_ = nullptr;
    on_ = false;
  }
  KernelTimer* tm_;
  int id_;
  bool on_ = false;
  hipEvent_t a_ = nullptr, b_ = nullptr;
};

// Everything one forward launch needs (device pointers).
struct FwdLaunch {
  int precision;
  bool io_bf16;
  bool single_seq;               // one sequence: tile order is computed in-kernel
  int head_dim, n_heads_q, n_heads_kv, total_tokens;
  int n_tiles;
  // query rows per workgroup of the bf16 forward: 64, or 32 or 16 (two or
  // four workgroups per tile) for launches that would otherwise leave CUs idle
  int tile_rows;
  float scale_log2;
  const void *q, *k, *v;
  void *out, *q_rot, *k_rot;
  float* lse;
  void* kc;                      // rotated K in the compute dtype (may be k_rot)
  void* vc;                      // V in the compute dtype when it differs from v's, else null
  const TileDesc* tiles_fwd;     // longest query tiles first
  const int32_t* pos_of;         // position of each token inside its sequence
  const float *cos_t, *sin_t;    // [max len][D/2]
};

// Backward kernel choice for bf16 tensors.  kBwdAuto takes the 32x32x16-MFMA
// kernel (attn_bwd3.hip) once the call's work, query heads times causal pairs
// per head, reaches the measured break-even below, the 16-row-wave kernel
// (attn_kernels.hip) under it: the wide kernel's extra row-stats launch, its
// larger per-workgroup fixed costs and its 128-row tiles (fewer workgroups)
// only pay off on large calls.  Steady-state fwd+bwd steps, both kernels
// pinned: D=128 the 16-row kernel ahead up to 23e6 (28/4 heads at S=1280)
// and the wide one from 33e6 (S=1536; two 1024-token sequences at 32/8
// heads); D=64 the 16-row kernel ahead up to 117e6 (14/2 heads at S=4096),
// the wide one from 132e6 (28/4 heads at S=3072), within 1% between.  The
// 32-row-wave kernel (attn_bwd.hip), slower than the wide one at every length
// measured, runs only when pinned.
enum BwdVariant : int { kBwdAuto = 0, kBwdRows16 = 1, kBwdRows32 = 2, kBwdMfma32 = 3 };
constexpr long long kBwdMfma32MinWorkD128 = 29000000LL;
constexpr long long kBwdMfma32MinWorkD64 = 125000000LL;

struct BwdLaunch {
  int precision;
  bool io_bf16;
  bool single_seq;               // one sequence: tile order is computed in-kernel
  int variant;                   // BwdVariant
  int head_dim, n_heads_q, n_heads_kv, total_tokens;
  int n_tiles;
  long long pairs;               // causal (query, key) pairs per head: sum L (L + 1) / 2
  float scale_log2, scale;
  const void *d_out, *q_rot, *k_rot, *v, *out;
  const float* lse;
  void *dq, *dk, *dv;
  void *wk, *wv;                 // per-query-head dK/dV partials [T][Hq][D], tensors' dtype
  void* stats;                   // bf16 tensors: [Hq][T] float2 (-lse log2 e, dO . O)
  const TileDesc* tiles_bwd;     // [2 n_tiles] dK/dV and dQ tiles, longest expected first
  // Split dK/dV tiles (16-row backward only; split == 0: none): the table
  // with dK/dV tiles 0 .. split - 1 of every sequence in halves, its length,
  // and the second halves' partials [T][Hq][D] (rows of split tiles only).
  int split;
  int n_split_entries;
  const TileDesc* tiles_split;
  void *wk2, *wv2;
  // The 128-row tile table of the 32x32x16-MFMA backward (null: not built;
  // that kernel is then not used) and its length.
  const TileDesc* tiles_wide;
  int n_wide_entries;
  // That kernel's workgroups take two query heads of a group each: a dK/dV
  // tile walks both into one partial (the head reduction then sums every
  // second head), a dQ tile runs both heads' tiles in turn.
  bool dkdv_head_pairs;
  const int32_t* pos_of;
  const float *cos_t, *sin_t;
};

// How many dK/dV tiles per sequence the backward splits (see TileKind): the
// largest split <= kBwdMaxSplit for which Hq workgroups per table entry
// still fit n_cu with an eighth to spare (a few more workgroups than CUs
// still shorten the span: the short tiles fill in behind), for bf16 tensors;
// 0 for fp32 tensors.  tiles_of(b) gives the tile count of sequence b of
// n_seqs.
template <typename F>
int bwd_split_of(bool io_bf16, int n_heads_q, int n_seqs, int n_cu, F tiles_of) {
  if (!io_bf16) return 0;
  long long base = 0;
  for (int b = 0; b < n_seqs; ++b) base += 2LL * tiles_of(b);
  int best = 0;
  for (int s = 1; s <= kBwdMaxSplit; ++s) {
    long long entries = base;
    for (int b = 0; b < n_seqs; ++b) entries += std::min(s, tiles_of(b));
    if ((long long)n_heads_q * entries <= n_cu + n_cu / 8) best = s;
  }
  return best;
}

// Queries of a dK/dV tile entry: query tiles [first, end) of a sequence with
// ntq tiles.
struct QueryRange {
  int first, end;
};
__host__ __device__ inline QueryRange dkdv_query_range(int tile, int ntq, int kind) {
  const int mid = tile + (ntq - tile + 1) / 2;
  if (kind == kTileDkDvFirstHalf) return QueryRange{tile, mid};
  if (kind == kTileDkDvSecondHalf) return QueryRange{mid, ntq};
  return QueryRange{tile, ntq};
}

hipError_t launch_forward(const FwdLaunch& a, hipStream_t st, KernelTimer* tm);
hipError_t launch_backward(const BwdLaunch& a, hipStream_t st, KernelTimer* tm);
size_t compute_elem_size(int precision, bool io_bf16);

// The bf16-MFMA attention forward (attn_fwd.hip), after rope_k has written
// the rotated K (and bf16 V) it reads.  IO: the dtype of q, out and q_rot
// (__bf16 or float); D: 64 or 128.
template <typename IO, int D>
hipError_t launch_fwd_bf16(const FwdLaunch& a, hipStream_t st, KernelTimer* tm);

// The bf16-tensor backward (attn_bwd.hip): the row-stats kernel and the
// dK/dV + dQ kernel, writing dq and the per-head dK/dV partials; D: 64 or 128.
template <int D>
hipError_t launch_bwd2(const BwdLaunch& a, hipStream_t st, KernelTimer* tm);

// The bf16-tensor backward on 32x32x16 MFMAs (attn_bwd3.hip): its row-stats
// kernel and the dK/dV + dQ kernel, writing dq and the per-head dK/dV
// partials; D: 64 or 128.
template <int D>
hipError_t launch_bwd3(const BwdLaunch& a, hipStream_t st, KernelTimer* tm);

// Head sizes the kernels are not built for (attn_pad.hip): rows of d
// elements padded to dp (a built size) with the rotation halves kept apart
// (columns 0 .. d/2 - 1 and dp/2 .. dp/2 + d/2 - 1, an odd d's last element
// at d/2, zeros elsewhere), and back; rows: tokens x heads; bf16 or float.
hipError_t launch_pad_rows(bool io_bf16, const void* src, void* dst, long rows, int d, int dp,
                           hipStream_t st);
hipError_t launch_unpad_rows(bool io_bf16, const void* src, void* dst, long rows, int d, int dp,
                             hipStream_t st);

// Kernels whose dynamic LDS exceeds 64 KB must say so before their launch.
template <typename F>
hipError_t allow_lds(F* fn, size_t bytes) {
  if (bytes <= 65536) return hipSuccess;
  return hipFuncSetAttribute(reinterpret_cast<const void*>(fn),
                             hipFuncAttributeMaxDynamicSharedMemorySize,
                             static_cast<int>(bytes));
}

// A kernel launch on st: with t's events when timing is on
// (hipExtLaunchKernelGGL), else a plain launch that stream capture records
// like any other.  KERNEL in parentheses when it has template arguments.
#define GL_LAUNCH(t, KERNEL, grid, block, lds, st, ...)                                        \
  do {                                                                                      \
    if ((t).start() != nullptr)                                                             \
      hipExtLaunchKernelGGL(KERNEL, grid, block, lds, st, (t).start(), (t).stop(), 0, __VA_ARGS__); \
    else                                                                                    \
      hipLaunchKernelGGL(KERNEL, grid, block, lds, st, __VA_ARGS__);                        \
  } while (0)

#define GL_CHECK(expr)               \
  do {                               \
    hipError_t e_ = (expr);          \
    if (e_ != hipSuccess) return e_; \
  } while (0)

}  // namespace glacier
