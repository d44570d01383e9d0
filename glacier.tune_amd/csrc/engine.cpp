// engine.cpp -- host side of libglacier_attn.so.
//
// GpuAttentionEngine mirrors the attention half of Glacier.Tune's
// GpuLoraEngine (src/Glacier.Tune/Gpu/GpuLoraEngine*.cs): the same entry
// points (SupportsAttention, ForwardAttention, BackwardAttention), the same
// argument meaning and the same error behaviour (bad arguments are rejected
// before any device work, device failures surface as errors, scratch grows
// on demand and is never shrunk, one call at a time per engine).  The
// extern "C" functions at the bottom are the C ABI declared in
// include/glacier_attn.h; they translate exceptions into status codes.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <map>
#include <memory>
#include <mutex>
#include <stdexcept>
#include <string>
#include <vector>

#include "../../include/glacier_attn.h"
#include "../../include/glacier_lmhead.h"
#include "../../include/glacier_norm.h"
#include "../../include/glacier_qkv.h"
#include "attn_launch.hpp"
#include "blas_lt.hpp"
#include "lmhead_launch.hpp"
#include "lora_file.hpp"
#include "noalloc.hpp"
#include "norm_launch.hpp"
#include "proj_launch.hpp"

namespace glacier {

namespace {

thread_local std::string g_last_error;

class Error : public std::runtime_error {
 public:
  Error(int code, const std::string& msg) : std::runtime_error(msg), code_(code) {}
  int code() const { return code_; }

 private:
  int code_;
};

[[noreturn]] void fail(int code, const std::string& msg) { throw Error(code, msg); }

void check_hip(hipError_t e, const char* what) {
  if (e == hipSuccess) return;
  if (e == hipErrorOutOfMemory || e == hipErrorMemoryAllocation)
    fail(GLACIER_ATTN_ERR_OUT_OF_MEMORY, std::string(what) + ": " + hipGetErrorString(e));
  fail(GLACIER_ATTN_ERR_DEVICE, std::string(what) + ": " + hipGetErrorString(e));
}

// Device allocation that only grows (x2 on growth), like the capacity
// fields of GpuLoraEngine.EnsureAttnCapacity (GpuLoraEngine.Memory.cs:60-114).
struct DeviceBuffer {
  void* ptr = nullptr;
  size_t cap = 0;
  ~DeviceBuffer() { release(); }
  void release() {
    if (ptr != nullptr) (void)hipFree(ptr);
    ptr = nullptr;
    cap = 0;
  }
  void* ensure(size_t bytes, const char* what) {
    if (bytes <= cap && ptr != nullptr) return ptr;
    release();
    size_t want = std::max<size_t>(bytes * 2, 256);
    hipError_t e = hipMalloc(&ptr, want);
    if (e != hipSuccess) {
      ptr = nullptr;
      (void)hipGetLastError();
      fail(GLACIER_ATTN_ERR_OUT_OF_MEMORY,
           std::string("hipMalloc(") + what + ", " + std::to_string(want) + " bytes): " +
               hipGetErrorString(e));
    }
    cap = want;
    return ptr;
  }
};

struct Shape {
  int total_tokens = 0;
  int n_heads_q = 0, n_heads_kv = 0, head_dim = 0;
  int real_dim = 0;  // the call's head size when head_dim is its padded one (0: head_dim)
  float rope_freq_base = 0.0f;
  int precision = 0;
  bool io_bf16 = false;
  std::vector<int32_t> cu;  // n_seqs + 1 offsets
};

// A validated call shape that points at the caller's cu_seqlens instead of
// copying it (the allocation-free entry point builds no host containers).
struct ShapeArgs {
  int total_tokens = 0, n_seqs = 1;
  const int32_t* cu = nullptr;  // nullptr: one sequence of total_tokens
  int n_heads_q = 0, n_heads_kv = 0, head_dim = 0;
  float rope_freq_base = 0.0f;
  int precision = 0;
  bool io_bf16 = false;
  int max_len = 0;
  int seq_start(int b) const { return cu != nullptr ? cu[b] : (b == 0 ? 0 : total_tokens); }
};

// Shape part of one backward launch.
struct BwdCall {
  int total_tokens, n_heads_q, n_heads_kv, head_dim, precision;
  bool io_bf16, single_seq;
  int n_tiles;
  long long pairs;
};

// RoPE angle of pair i at position pos: the fp32 operations of
// RoPEKernel.cs:64-68 (glibc powf, then cosf/sinf of pos * freq).
inline float rope_freq(int i, int head_dim, float base) {
  return 1.0f / powf(base, static_cast<float>(2 * i) / static_cast<float>(head_dim));
}

// Backward dK/dV and dQ tiles of one sequence layout in launch order, longest
// expected first (list scheduling: the long tiles of both kinds start at once
// and the short ones fill the tail).  The cost is linear in the tile pairs a
// tile visits, with constants fitted to measured workgroup durations (D = 128,
// units of 0.1 us); it only orders the launch.
inline int bwd_tile_cost(int n_tiles_in_seq, int tile, int kind) {
  if (kind == kTileDq) return 53 + 12 * (tile + 1);
  const QueryRange r = dkdv_query_range(tile, n_tiles_in_seq, kind);
  return 63 + 16 * (r.end - r.first);
}

// Expected cost of a 128-row backward tile (attn_bwd3.hip) of a sequence of
// len tokens: its step count (one per 32-row chunk it visits, plus one),
// weighted by the step time of its kind, plus a fixed part; it only orders
// the launch.
inline int bwd_wide_cost(int len, int tile, int kind, bool head_pairs) {
  if (kind == kTileDq || kind == kTileDqSecond) {
    const int keys = std::min(len, kWideTile * (tile + 1));
    return 50 + 18 * (((keys + 31) / 32 + 1) / 2 + 1);
  }
  // a dK/dV tile over a head pair walks twice the query chunks
  return 50 + (head_pairs ? 24 : 12) * ((len - kWideTile * tile + 31) / 32 + 1);
}

// The wide backward's entries per 128-row tile: dK/dV and dQ, plus the dQ
// tile of a head pair's second head when its workgroups take head pairs.
inline std::vector<int> wide_kinds(bool head_pairs) {
  if (head_pairs) return {kTileDkDv, kTileDq, kTileDqSecond};
  return {kTileDkDv, kTileDq};
}

// The backward entries of one sequence of nt tiles in natural order (tile by
// tile, dK/dV before dQ); the dK/dV tiles below `split` come as two halves.
template <typename F>
void bwd_entries(int nt, int split, F emit) {
  for (int t = 0; t < nt; ++t) {
    if (t < split) {
      emit(t, static_cast<int>(kTileDkDvFirstHalf));
      emit(t, static_cast<int>(kTileDkDvSecondHalf));
    } else {
      emit(t, static_cast<int>(kTileDkDv));
    }
    emit(t, static_cast<int>(kTileDq));
  }
}

// ---- allocation-free backward: its buffers inside the fixed scratch -------
constexpr int kNoAllocMaxSeqs = 1024;
constexpr int kNoAllocMaxTokens = GLACIER_ATTN_MAX_SEQ_LEN;
constexpr int kNoAllocMaxTiles = kNoAllocMaxTokens / kTile + kNoAllocMaxSeqs;
constexpr int kNoAllocMaxCost = 63 + 16 * (kNoAllocMaxTokens / kTile);
constexpr int kNoAllocMaxSplitEntries = 4096;  // a split table fits the CUs: far fewer
// the 128-row table of the wide backward: two entries per 128-row tile
constexpr int kNoAllocMaxWideEntries = 2 * (kNoAllocMaxTokens / kWideTile + kNoAllocMaxSeqs);
constexpr int kNoAllocMaxWideCost = 50 + 24 * ((kNoAllocMaxTokens + 31) / 32 + 1);
constexpr int kNoAllocRopeChunk = 16384;  // floats staged per table upload

// What one device's scratch holds across calls: the RoPE tables and the tile
// and position tables of the last sequence layout.
struct NoAllocResident {
  int rope_cap = 0, rope_dim = 0;
  float rope_base = 0.0f;
  size_t tiles_off = 0;  // 0: no tile table resident
  int n_seqs = 0, total_tokens = 0, split = 0, n_wide = 0;
  int32_t cu[kNoAllocMaxSeqs + 1] = {};
};

std::mutex g_noalloc_mutex;  // guards the records and host staging below
NoAllocResident g_noalloc[kNoAllocMaxDevices];
TileDesc g_noalloc_tiles[2 * kNoAllocMaxTiles + kNoAllocMaxSplitEntries + kNoAllocMaxWideEntries];
int32_t g_noalloc_pos[kNoAllocMaxTokens];
int32_t g_noalloc_count[(kNoAllocMaxCost > kNoAllocMaxWideCost ? kNoAllocMaxCost : kNoAllocMaxWideCost) + 2];
float g_noalloc_freq[512];  // head_dim / 2 (head_dim <= 1024, make_shape_args)
float g_noalloc_stage[kNoAllocRopeChunk];

size_t align256(size_t x) { return (x + 255) & ~static_cast<size_t>(255); }

struct NoAllocBwd {
  void *wk, *wv, *stats;
  const TileDesc* tiles_bwd;
  int split, n_split_entries;  // split dK/dV tiles (split > 0): their table and partials
  const TileDesc* tiles_split;
  void *wk2, *wv2;
  const TileDesc* tiles_wide;  // the wide backward's table (null: not built)
  int n_wide_entries;
  const int32_t* pos_of;
  const float *cos_t, *sin_t;
  int n_tiles;
  long long pairs;
};

// Lays out one backward call inside the scratch at `base` on `device`:
//   [cos table][sin table][dK/dV + dQ tile table, the split table, the wide table][positions]
//   [row stats]
//   [dK partials][dV partials][second-half dK partials][second-half dV partials]
// (each region 256-byte aligned; the split regions only when the call splits
// dK/dV tiles, by the rule of the allocating backward: bwd_split_of with the
// device's n_cu, unless split_ok is false).  The RoPE tables and the tile/position
// tables are uploaded only when the call's head_dim, theta, longest sequence
// or sequence layout differ from what the scratch holds; the upload first
// waits for the whole device, since any earlier call may still read them.
// Every other region is written by the call's own kernels before it is read.
NoAllocBwd noalloc_bwd_workspace(int device, void* base, const ShapeArgs& s, int n_cu,
                                 bool split_ok, bool head_pairs) {
  if (s.n_seqs > kNoAllocMaxSeqs)
    fail(GLACIER_ATTN_ERR_UNSUPPORTED, "the allocation-free backward takes at most " +
                                           std::to_string(kNoAllocMaxSeqs) + " sequences per call");
  if (s.total_tokens > kNoAllocMaxTokens)
    fail(GLACIER_ATTN_ERR_UNSUPPORTED, "the allocation-free backward takes at most " +
                                           std::to_string(kNoAllocMaxTokens) + " tokens per call");
  const size_t T = s.total_tokens, Hq = s.n_heads_q, D = s.head_dim;
  const int half = s.head_dim / 2;
  int n_tiles = 0;
  long long pairs = 0;
  for (int b = 0; b < s.n_seqs; ++b) {
    const int len = s.seq_start(b + 1) - s.seq_start(b);
    n_tiles += (len + kTile - 1) / kTile;
    pairs += static_cast<long long>(len) * (len + 1) / 2;
  }
  auto tiles_of = [&](int b) { return (s.seq_start(b + 1) - s.seq_start(b) + kTile - 1) / kTile; };
  int split = split_ok ? bwd_split_of(s.io_bf16, s.n_heads_q, s.n_seqs, n_cu, tiles_of) : 0;
  int n_split_entries = 0;
  if (split > 0) {
    n_split_entries = 2 * n_tiles;
    for (int b = 0; b < s.n_seqs; ++b) n_split_entries += std::min(split, tiles_of(b));
    if (n_split_entries > kNoAllocMaxSplitEntries) split = n_split_entries = 0;
  }
  std::lock_guard<std::mutex> g(g_noalloc_mutex);
  NoAllocResident& r = g_noalloc[device];
  const bool rope_ok = r.rope_cap >= s.max_len && r.rope_dim == s.head_dim &&
                       r.rope_base == s.rope_freq_base;
  const int rope_cap = rope_ok ? r.rope_cap : (std::max(s.max_len, 1) + 255) / 256 * 256;
  const size_t rope_bytes = align256(static_cast<size_t>(rope_cap) * half * sizeof(float));
  const size_t off_tiles = 2 * rope_bytes;
  // the wide backward's table, for the tensors and head sizes it takes
  int n_wide = 0;
  const std::vector<int> wkinds = wide_kinds(head_pairs);
  const int per_wide = static_cast<int>(wkinds.size());  // entries per 128-row tile
  if (s.io_bf16 && (s.head_dim == 64 || s.head_dim == 128))
    for (int b = 0; b < s.n_seqs; ++b)
      n_wide += per_wide * ((s.seq_start(b + 1) - s.seq_start(b) + kWideTile - 1) / kWideTile);
  const size_t n_entries = 2 * static_cast<size_t>(n_tiles) + n_split_entries + n_wide;
  const size_t off_pos = off_tiles + align256(n_entries * sizeof(TileDesc));
  const size_t off_stats = off_pos + align256(T * sizeof(int32_t));
  const size_t stats_bytes = s.io_bf16 ? align256((T * Hq + 64) * 2 * sizeof(float)) : 0;
  const size_t part = align256(T * Hq * D * (s.io_bf16 ? 2 : 4));
  const size_t off_wk = off_stats + stats_bytes, off_wv = off_wk + part;
  const size_t off_wk2 = off_wv + part, off_wv2 = off_wk2 + (split > 0 ? part : 0);
  const size_t need = off_wv2 + (split > 0 ? part : 0);
  if (need > kNoAllocScratchBytes)
    fail(GLACIER_ATTN_ERR_UNSUPPORTED,
         "the allocation-free backward needs " + std::to_string(need) +
             " bytes of scratch for this call; its fixed scratch holds " +
             std::to_string(kNoAllocScratchBytes) + " (GLACIER_ATTN_NOALLOC_SCRATCH_BYTES)");
  bool tiles_ok = r.tiles_off == off_tiles && r.n_seqs == s.n_seqs &&
                  r.total_tokens == s.total_tokens && r.split == split && r.n_wide == n_wide;
  for (int b = 0; tiles_ok && b <= s.n_seqs; ++b) tiles_ok = r.cu[b] == s.seq_start(b);
  char* const sb = static_cast<char*>(base);
  if (!rope_ok || !tiles_ok) {
    check_hip(hipDeviceSynchronize(), "allocation-free backward: wait before a table update");
    if (!rope_ok) {
      r.rope_cap = 0;
      for (int i = 0; i < half; ++i) g_noalloc_freq[i] = rope_freq(i, s.head_dim, s.rope_freq_base);
      const int rows = kNoAllocRopeChunk / half;
      for (int table = 0; table < 2; ++table) {
        for (int p0 = 0; p0 < rope_cap; p0 += rows) {
          const int p1 = std::min(rope_cap, p0 + rows);
          for (int pos = p0; pos < p1; ++pos)
            for (int i = 0; i < half; ++i) {
              const float theta = static_cast<float>(pos) * g_noalloc_freq[i];
              g_noalloc_stage[(pos - p0) * half + i] = table == 0 ? cosf(theta) : sinf(theta);
            }
          check_hip(hipMemcpy(sb + table * rope_bytes + static_cast<size_t>(p0) * half * sizeof(float),
                              g_noalloc_stage, static_cast<size_t>(p1 - p0) * half * sizeof(float),
                              hipMemcpyHostToDevice),
                    "allocation-free backward: RoPE table upload");
        }
      }
      r.rope_cap = rope_cap;
      r.rope_dim = s.head_dim;
      r.rope_base = s.rope_freq_base;
    }
    if (!tiles_ok) {
      r.tiles_off = 0;
      // stable counting sort of the tiles (natural order: sequence, tile,
      // dK/dV before dQ) by expected cost, longest first
      std::fill(g_noalloc_count, g_noalloc_count + kNoAllocMaxCost + 2, 0);
      for (int b = 0; b < s.n_seqs; ++b) {
        const int len = s.seq_start(b + 1) - s.seq_start(b);
        const int nt = (len + kTile - 1) / kTile;
        for (int t = 0; t < nt; ++t)
          for (int kind = 0; kind < 2; ++kind) ++g_noalloc_count[bwd_tile_cost(nt, t, kind)];
      }
      int next = 0;
      for (int c = kNoAllocMaxCost; c >= 0; --c) {
        const int n = g_noalloc_count[c];
        g_noalloc_count[c] = next;
        next += n;
      }
      for (int b = 0; b < s.n_seqs; ++b) {
        const int tok0 = s.seq_start(b), len = s.seq_start(b + 1) - tok0;
        const int nt = (len + kTile - 1) / kTile;
        for (int t = 0; t < nt; ++t)
          for (int kind = 0; kind < 2; ++kind)
            g_noalloc_tiles[g_noalloc_count[bwd_tile_cost(nt, t, kind)]++] =
                TileDesc{tok0, len, t, kind};
        for (int i = 0; i < len; ++i) g_noalloc_pos[tok0 + i] = i;
      }
      if (split > 0) {
        // the split table: the same stable counting sort over the entries
        // with dK/dV tiles 0 .. split - 1 in halves
        TileDesc* const out = g_noalloc_tiles + 2 * n_tiles;
        std::fill(g_noalloc_count, g_noalloc_count + kNoAllocMaxCost + 2, 0);
        for (int b = 0; b < s.n_seqs; ++b) {
          const int nt = tiles_of(b);
          bwd_entries(nt, split, [&](int t, int kind) { ++g_noalloc_count[bwd_tile_cost(nt, t, kind)]; });
        }
        int at = 0;
        for (int c = kNoAllocMaxCost; c >= 0; --c) {
          const int n = g_noalloc_count[c];
          g_noalloc_count[c] = at;
          at += n;
        }
        for (int b = 0; b < s.n_seqs; ++b) {
          const int tok0 = s.seq_start(b), len = s.seq_start(b + 1) - tok0, nt = tiles_of(b);
          bwd_entries(nt, split, [&](int t, int kind) {
            out[g_noalloc_count[bwd_tile_cost(nt, t, kind)]++] = TileDesc{tok0, len, t, kind};
          });
        }
      }
      if (n_wide > 0) {
        // the wide table: the same stable counting sort by bwd_wide_cost
        TileDesc* const out = g_noalloc_tiles + 2 * n_tiles + n_split_entries;
        std::fill(g_noalloc_count, g_noalloc_count + kNoAllocMaxWideCost + 2, 0);
        for (int b = 0; b < s.n_seqs; ++b) {
          const int len = s.seq_start(b + 1) - s.seq_start(b);
          for (int t = 0; t < (len + kWideTile - 1) / kWideTile; ++t)
            for (int kind : wkinds) ++g_noalloc_count[bwd_wide_cost(len, t, kind, head_pairs)];
        }
        int at = 0;
        for (int c = kNoAllocMaxWideCost; c >= 0; --c) {
          const int n = g_noalloc_count[c];
          g_noalloc_count[c] = at;
          at += n;
        }
        for (int b = 0; b < s.n_seqs; ++b) {
          const int tok0 = s.seq_start(b), len = s.seq_start(b + 1) - tok0;
          for (int t = 0; t < (len + kWideTile - 1) / kWideTile; ++t)
            for (int kind : wkinds)
              out[g_noalloc_count[bwd_wide_cost(len, t, kind, head_pairs)]++] = TileDesc{tok0, len, t, kind};
        }
      }
      check_hip(hipMemcpy(sb + off_tiles, g_noalloc_tiles, n_entries * sizeof(TileDesc),
                          hipMemcpyHostToDevice),
                "allocation-free backward: tile table upload");
      check_hip(hipMemcpy(sb + off_pos, g_noalloc_pos, T * sizeof(int32_t), hipMemcpyHostToDevice),
                "allocation-free backward: position table upload");
      r.n_seqs = s.n_seqs;
      r.total_tokens = s.total_tokens;
      r.split = split;
      r.n_wide = n_wide;
      for (int b = 0; b <= s.n_seqs; ++b) r.cu[b] = s.seq_start(b);
      r.tiles_off = off_tiles;
    }
  }
  NoAllocBwd w{};
  w.cos_t = reinterpret_cast<const float*>(sb);
  w.sin_t = reinterpret_cast<const float*>(sb + rope_bytes);
  w.tiles_bwd = reinterpret_cast<const TileDesc*>(sb + off_tiles);
  w.pos_of = reinterpret_cast<const int32_t*>(sb + off_pos);
  w.stats = s.io_bf16 ? sb + off_stats : nullptr;
  w.wk = sb + off_wk;
  w.wv = sb + off_wv;
  w.split = split;
  w.n_split_entries = n_split_entries;
  w.tiles_split = split > 0 ? w.tiles_bwd + 2 * n_tiles : nullptr;
  w.wk2 = split > 0 ? sb + off_wk2 : nullptr;
  w.wv2 = split > 0 ? sb + off_wv2 : nullptr;
  w.tiles_wide = n_wide > 0 ? w.tiles_bwd + 2 * n_tiles + n_split_entries : nullptr;
  w.n_wide_entries = n_wide;
  w.n_tiles = n_tiles;
  w.pairs = pairs;
  return w;
}

// Tile lists of one sequence layout, resident on the device.
struct TileSet {
  int n_tiles = 0, max_len = 0;
  long long pairs = 0;  // causal (query, key) pairs per head
  // [3 n_tiles] TileDesc: fwd order, then the backward order; then, for
  // layouts small enough to split, the backward tables with split 1, 2, ...
  DeviceBuffer tiles;
  int split_at[kBwdMaxSplit + 1] = {};       // entry offset of each split table (0: none)
  int split_entries[kBwdMaxSplit + 1] = {};  // and its length
  int wide_at = 0, wide_entries = 0;         // the 128-row backward table (attn_bwd3.hip)
  int wide2_at = 0, wide2_entries = 0;       // the same over query-head pairs
  int wide_tiles = 0;                        // 128-row tiles: sum of ceil(len / 128)
  std::vector<int> seq_tiles;                // tiles of each sequence
  DeviceBuffer pos;    // [T] int32
};

}  // namespace

class GpuAttentionEngine {
 public:
  GpuAttentionEngine(int device_ordinal, int precision)
      : device_(device_ordinal), precision_(precision) {
    int n = 0;
    check_hip(hipGetDeviceCount(&n), "hipGetDeviceCount");
    if (device_ordinal < 0 || device_ordinal >= n)
      fail(GLACIER_ATTN_ERR_INVALID_ARGUMENT,
           "device ordinal " + std::to_string(device_ordinal) + " out of range (" +
               std::to_string(n) + " devices)");
    check_hip(hipSetDevice(device_), "hipSetDevice");
    check_hip(hipDeviceGetAttribute(&n_cu_, hipDeviceAttributeMultiprocessorCount, device_),
              "hipDeviceGetAttribute");
    check_hip(hipStreamCreateWithFlags(&own_stream_, hipStreamNonBlocking), "hipStreamCreate");
    // the allocation-free backward's scratch address on this device; a
    // failure here only disables that entry point (it retries and reports)
    if (noalloc_scratch_init(device_) != hipSuccess) (void)hipGetLastError();
    // GLACIER_ATTN_BWD=rows16|rows32|mfma32 pins the bf16 backward kernel
    // (tests cover each on every shape); unset or "auto" picks by sequence
    // length.
    if (const char* v = std::getenv("GLACIER_ATTN_BWD")) {
      const std::string m(v);
      if (m == "rows16") bwd_variant_ = kBwdRows16;
      else if (m == "rows32") bwd_variant_ = kBwdRows32;
      else if (m == "mfma32") bwd_variant_ = kBwdMfma32;
      else if (m != "auto" && !m.empty())
        fail(GLACIER_ATTN_ERR_INVALID_ARGUMENT,
             "GLACIER_ATTN_BWD must be auto, rows16, rows32 or mfma32, not " + m);
    }
    // GLACIER_ATTN_BWD_SPLIT=0 keeps every dK/dV tile whole (comparisons and
    // A/B runs); unset or "auto" splits the longest ones when the CUs allow.
    if (const char* v = std::getenv("GLACIER_ATTN_BWD_SPLIT")) {
      const std::string m(v);
      if (m == "0") split_ok_ = false;
      else if (m != "auto" && !m.empty())
        fail(GLACIER_ATTN_ERR_INVALID_ARGUMENT,
             "GLACIER_ATTN_BWD_SPLIT must be auto or 0, not " + m);
    }
    // GLACIER_ATTN_BWD_PAIRS=1 makes the wide backward's workgroups take two
    // query heads of a group each (one dK/dV partial per head pair), 0 one;
    // unset or "auto" decides per call (head_pairs_for).
    if (const char* v = std::getenv("GLACIER_ATTN_BWD_PAIRS")) {
      const std::string m(v);
      if (m == "1") bwd_pairs_mode_ = 1;
      else if (m == "0") bwd_pairs_mode_ = 0;
      else if (m != "auto" && !m.empty())
        fail(GLACIER_ATTN_ERR_INVALID_ARGUMENT,
             "GLACIER_ATTN_BWD_PAIRS must be auto, 0 or 1, not " + m);
    }
    // GLACIER_ATTN_FWD_ROWS=16|32|64 pins the bf16 forward's query rows per
    // workgroup; unset or "auto" decides per call (fwd_rows_for).
    if (const char* v = std::getenv("GLACIER_ATTN_FWD_ROWS")) {
      const std::string m(v);
      if (m == "32") fwd_rows_ = 32;
      else if (m == "16") fwd_rows_ = 16;
      else if (m == "64") fwd_rows_ = 64;
      else if (m != "auto" && !m.empty())
        fail(GLACIER_ATTN_ERR_INVALID_ARGUMENT,
             "GLACIER_ATTN_FWD_ROWS must be auto, 16, 32 or 64, not " + m);
    }
  }

  ~GpuAttentionEngine() {
    (void)hipSetDevice(device_);
    if (own_stream_ != nullptr) (void)hipStreamSynchronize(own_stream_);
    if (blas_ != nullptr) {
      // GEMMs may still run on a caller's stream with the handle's workspace
      (void)hipDeviceSynchronize();
      destroy_blas_handle(blas_);
    }
    if (own_stream_ != nullptr) (void)hipStreamDestroy(own_stream_);
  }

  // GpuLoraEngine.SupportsAttention (GpuLoraEngine.cs:111-112): the shapes
  // the GPU kernels take; anything else stays on the CPU path.
  static bool SupportsAttention(int seq_len, int head_dim) {
    return SupportedHeadDim(head_dim) && seq_len >= 1 && seq_len <= GLACIER_ATTN_MAX_SEQ_LEN;
  }
  // The kernels are built for head sizes 32, 64, 96, 128 and 256; any other
  // size from 1 to 256 runs them on rows padded to the next of those.
  static bool SupportedHeadDim(int d) { return d >= 1 && d <= 256; }
  static int PaddedHeadDim(int d) {
    for (int n : {32, 64, 96, 128, 256})
      if (d <= n) return n;
    return 0;
  }

  std::mutex& lock() { return mutex_; }
  hipStream_t stream() const { return has_user_stream_ ? user_stream_ : own_stream_; }
  void set_stream(hipStream_t s) {
    user_stream_ = s;
    has_user_stream_ = true;
  }
  void use_own_stream() { has_user_stream_ = false; }
  int precision() const { return precision_; }
  KernelTimer& timer() { return timer_; }
  void activate() { check_hip(hipSetDevice(device_), "hipSetDevice"); }

  // ---- device entry points --------------------------------------------
  // LaunchRopeBatch + LaunchAttnTrainFwd (GpuLoraEngine.Forward.cs:401-465).
  void LaunchAttnTrainFwd(const Shape& s, const void* q, const void* k, const void* v,
                          void* out, float* lse, void* q_rot, void* k_rot) {
    if (s.total_tokens == 0) return;
    const int dp = PaddedHeadDim(s.head_dim);
    if (dp != s.head_dim) {
      // a head size the kernels are not built for: padded rows (attn_pad.hip)
      const bool bf = s.io_bf16;
      const long rq = (long)s.total_tokens * s.n_heads_q, rk = (long)s.total_tokens * s.n_heads_kv;
      const int d = s.head_dim;
      const size_t esz = bf ? 2 : 4;
      void* qp = pad_q_.ensure(rq * dp * esz, "padded q");
      void* kp = pad_k_.ensure(rk * dp * esz, "padded k");
      void* vp = pad_v_.ensure(rk * dp * esz, "padded v");
      void* op = pad_o_.ensure(rq * dp * esz, "padded out");
      void* qrp = q_rot != nullptr ? pad_qr_.ensure(rq * dp * esz, "padded q_rot") : nullptr;
      void* krp = k_rot != nullptr ? pad_kr_.ensure(rk * dp * esz, "padded k_rot") : nullptr;
      check_hip(launch_pad_rows(bf, q, qp, rq, d, dp, stream()), "pad q");
      check_hip(launch_pad_rows(bf, k, kp, rk, d, dp, stream()), "pad k");
      check_hip(launch_pad_rows(bf, v, vp, rk, d, dp, stream()), "pad v");
      Shape sp = s;
      sp.head_dim = dp;
      sp.real_dim = d;
      LaunchAttnTrainFwd(sp, qp, kp, vp, op, lse, qrp, krp);
      check_hip(launch_unpad_rows(bf, op, out, rq, d, dp, stream()), "unpad out");
      if (q_rot != nullptr) check_hip(launch_unpad_rows(bf, qrp, q_rot, rq, d, dp, stream()), "unpad q_rot");
      if (k_rot != nullptr) check_hip(launch_unpad_rows(bf, krp, k_rot, rk, d, dp, stream()), "unpad k_rot");
      return;
    }
    const int dreal = s.real_dim > 0 ? s.real_dim : s.head_dim;
    const TileSet& ts = tiles_for(s);
    EnsureRopeTable(ts.max_len, s.head_dim, s.rope_freq_base, dreal);
    const size_t esz = compute_elem_size(s.precision, s.io_bf16);
    const size_t io_esz = s.io_bf16 ? 2 : 4;
    FwdLaunch a{};
    a.precision = s.precision;
    a.io_bf16 = s.io_bf16;
    a.single_seq = s.cu.size() == 2;
    a.head_dim = s.head_dim;
    a.n_heads_q = s.n_heads_q;
    a.n_heads_kv = s.n_heads_kv;
    a.total_tokens = s.total_tokens;
    a.n_tiles = ts.n_tiles;
    a.tile_rows = fwd_rows_ != 0 ? fwd_rows_ : fwd_rows_for(s.n_heads_q, ts.n_tiles, s.head_dim);
    a.scale_log2 = kLog2e / std::sqrt(static_cast<float>(dreal));
    a.q = q; a.k = k; a.v = v;
    a.out = out; a.lse = lse; a.q_rot = q_rot; a.k_rot = k_rot;
    // The attention kernel reads rotated K in the compute dtype: the caller's
    // k_rot when it is that dtype, else library scratch.
    if (k_rot != nullptr && esz == io_esz)
      a.kc = k_rot;
    else
      a.kc = kc_.ensure((size_t)s.total_tokens * s.n_heads_kv * s.head_dim * esz, "K scratch");
    // bf16 matrix cores on fp32 tensors: rope_k also writes a bf16 copy of V.
    if (esz != io_esz)
      a.vc = vc_.ensure((size_t)s.total_tokens * s.n_heads_kv * s.head_dim * esz, "V scratch");
    const TileDesc* t = static_cast<const TileDesc*>(ts.tiles.ptr);
    a.tiles_fwd = t;
    a.pos_of = static_cast<const int32_t*>(ts.pos.ptr);
    a.cos_t = rope_cos();
    a.sin_t = rope_sin();
    check_hip(launch_forward(a, stream(), &timer_), "attention forward launch");
  }

  // Query rows per workgroup of the bf16 forward: 16 when those workgroups
  // still fit the chip at once (two per CU where head_dim 64 leaves room in
  // the LDS, one at 128), 32 when those fill at most one and a half rounds of
  // the CUs, else 64.  Measured (bench.py, one box): qwen05b S=512 forward
  // 9.5 -> 7.2 us at 32 rows -> 6.6-6.9 us at 16; where the 64-row grid
  // already fills the chip fewer rows are slower (qwen7b S=512: 13.3, 14.2
  // and 19.8 us at 64, 32 and 16 rows, its 32-row grid 1.75 rounds).  Steady-
  // state fwd+bwd steps at 1-1.5 rounds, 32 against 64 rows: 12/2 heads
  // S=1024 48.3 -> 47.0 us, 14/2 heads D=64 S=768 31.4 -> 30.1, 8/2 heads
  // S=1536 61.1 -> 57.7; 28/4 heads S=384 31.8 -> 32.1.
  int fwd_rows_for(int n_heads_q, int n_tiles, int head_dim) const {
    const long long units = static_cast<long long>(n_heads_q) * n_tiles;  // 64-row tiles
    const int per_cu = head_dim <= 64 ? 2 : 1;
    if (4 * units <= static_cast<long long>(per_cu) * n_cu_) return 16;
    if (4 * units <= 3LL * n_cu_) return 32;
    return 64;
  }

  // Whether the wide backward takes query heads in pairs.  Measured (one box,
  // backward calls): 32/8 heads, B=2 x S=1024 132 -> 120 us, B=2 x S=2048
  // 370 -> 337 us, S=4096 580 -> 551 us; slower where halving the dK/dV
  // workgroups leaves the chip short of them (16/2 heads at S=2048: 72 ->
  // 118 us).  An odd group leaves one head of every group alone (half-length
  // workgroups); fwd+bwd steps, two rounds: 28/4 heads D=128 S=2048 226 ->
  // 219 us, S=4096 646 -> 633, two sequences of 2048 even; but 14/2 heads
  // D=64 S=4096 254 -> 270, 40/8 heads S=4096 908 -> 955, and every shape
  // with fewer pair workgroups than CUs slower.  So: an even group with at
  // least one pair workgroup per CU, or a group of 7 or more heads at
  // D=128 with at least two per CU.
  bool head_pairs_for(int n_heads_q, int n_heads_kv, int head_dim, int wide_tiles) const {
    if (bwd_pairs_mode_ >= 0) return bwd_pairs_mode_ == 1;
    const int ratio = n_heads_q / n_heads_kv;
    const long long pair_wgs = static_cast<long long>((ratio + 1) / 2) * n_heads_kv * wide_tiles;
    if (ratio >= 2 && ratio % 2 == 0) return pair_wgs >= n_cu_;
    return ratio >= 7 && head_dim == 128 && pair_wgs >= 2LL * n_cu_;
  }

  // Shape part of a backward launch (pointers are filled by the caller).
  BwdLaunch bwd_launch_of(const BwdCall& c) const {
    BwdLaunch a{};
    a.precision = c.precision;
    a.io_bf16 = c.io_bf16;
    a.single_seq = c.single_seq;
    a.variant = bwd_variant_;
    a.head_dim = c.head_dim;
    a.n_heads_q = c.n_heads_q;
    a.n_heads_kv = c.n_heads_kv;
    a.total_tokens = c.total_tokens;
    a.n_tiles = c.n_tiles;
    a.pairs = c.pairs;
    a.scale = 1.0f / std::sqrt(static_cast<float>(c.head_dim));
    a.scale_log2 = kLog2e * a.scale;
    return a;
  }

  // LaunchAttnTrainBwd + inverse LaunchRopeBatch (GpuLoraEngine.Backward.cs:354-412, :452).
  void LaunchAttnTrainBwd(const Shape& s, const void* d_out, const void* q_rot,
                          const void* k_rot, const void* v, const void* out,
                          const float* lse, void* dq, void* dk, void* dv) {
    if (s.total_tokens == 0) return;
    const int dp = PaddedHeadDim(s.head_dim);
    if (dp != s.head_dim) {
      // a head size the kernels are not built for: padded rows (attn_pad.hip)
      const bool bf = s.io_bf16;
      const long rq = (long)s.total_tokens * s.n_heads_q, rk = (long)s.total_tokens * s.n_heads_kv;
      const int d = s.head_dim;
      const size_t esz = bf ? 2 : 4;
      void* dop = pad_do_.ensure(rq * dp * esz, "padded d_out");
      void* qrp = pad_qr_.ensure(rq * dp * esz, "padded q_rot");
      void* krp = pad_kr_.ensure(rk * dp * esz, "padded k_rot");
      void* vp = pad_v_.ensure(rk * dp * esz, "padded v");
      void* op = pad_o_.ensure(rq * dp * esz, "padded out");
      void* dqp = pad_dq_.ensure(rq * dp * esz, "padded dq");
      void* dkp = pad_dk_.ensure(rk * dp * esz, "padded dk");
      void* dvp = pad_dv_.ensure(rk * dp * esz, "padded dv");
      check_hip(launch_pad_rows(bf, d_out, dop, rq, d, dp, stream()), "pad d_out");
      check_hip(launch_pad_rows(bf, q_rot, qrp, rq, d, dp, stream()), "pad q_rot");
      check_hip(launch_pad_rows(bf, k_rot, krp, rk, d, dp, stream()), "pad k_rot");
      check_hip(launch_pad_rows(bf, v, vp, rk, d, dp, stream()), "pad v");
      check_hip(launch_pad_rows(bf, out, op, rq, d, dp, stream()), "pad out");
      Shape sp = s;
      sp.head_dim = dp;
      sp.real_dim = d;
      LaunchAttnTrainBwd(sp, dop, qrp, krp, vp, op, lse, dqp, dkp, dvp);
      check_hip(launch_unpad_rows(bf, dqp, dq, rq, d, dp, stream()), "unpad dq");
      check_hip(launch_unpad_rows(bf, dkp, dk, rk, d, dp, stream()), "unpad dk");
      check_hip(launch_unpad_rows(bf, dvp, dv, rk, d, dp, stream()), "unpad dv");
      return;
    }
    const int dreal = s.real_dim > 0 ? s.real_dim : s.head_dim;
    const TileSet& ts = tiles_for(s);
    EnsureRopeTable(ts.max_len, s.head_dim, s.rope_freq_base, dreal);
    const size_t T = s.total_tokens, Hq = s.n_heads_q, D = s.head_dim;
    BwdLaunch a = bwd_launch_of(BwdCall{s.total_tokens, s.n_heads_q, s.n_heads_kv, s.head_dim,
                                        s.precision, s.io_bf16, s.cu.size() == 2, ts.n_tiles,
                                        ts.pairs});
    a.scale = 1.0f / std::sqrt(static_cast<float>(dreal));
    a.scale_log2 = kLog2e * a.scale;
    a.d_out = d_out; a.q_rot = q_rot; a.k_rot = k_rot; a.v = v; a.out = out;
    a.lse = lse; a.dq = dq; a.dk = dk; a.dv = dv;
    // the per-head partials are kept in the tensors' dtype: bf16 tensors get
    // bf16 partials (half the traffic), fp32 tensors fp32 partials, so the
    // group reduction of the fp32-tensor entry points sums fp32 values
    const size_t wsz = s.io_bf16 ? 2 : 4;
    a.wk = wk_.ensure(T * Hq * D * wsz, "dK partials");
    a.wv = wv_.ensure(T * Hq * D * wsz, "dV partials");
    // bf16 tensors: the row stats [Hq][T] float2, plus 64 entries of padding
    // (the kernel reads them in blocks of 4 rows; rows past a sequence's end
    // are masked out, so the padding's contents never reach a result)
    if (s.io_bf16) a.stats = stats_.ensure((T * Hq + 64) * 2 * sizeof(float), "row stats");
    const TileDesc* t = static_cast<const TileDesc*>(ts.tiles.ptr);
    a.tiles_bwd = t + ts.n_tiles;
    a.dkdv_head_pairs = head_pairs_for(s.n_heads_q, s.n_heads_kv, s.head_dim, ts.wide_tiles);
    a.tiles_wide = t + (a.dkdv_head_pairs ? ts.wide2_at : ts.wide_at);
    a.n_wide_entries = a.dkdv_head_pairs ? ts.wide2_entries : ts.wide_entries;
    // the longest dK/dV tiles in query halves while the launch fits the CUs
    const int split =
        split_ok_ ? bwd_split_of(s.io_bf16, s.n_heads_q, static_cast<int>(ts.seq_tiles.size()),
                                 n_cu_, [&](int b) { return ts.seq_tiles[b]; })
                  : 0;
    if (split > 0 && ts.split_entries[split] > 0) {
      a.split = split;
      a.n_split_entries = ts.split_entries[split];
      a.tiles_split = t + ts.split_at[split];
      a.wk2 = wk2_.ensure(T * Hq * D * wsz, "second-half dK partials");
      a.wv2 = wv2_.ensure(T * Hq * D * wsz, "second-half dV partials");
    }
    a.pos_of = static_cast<const int32_t*>(ts.pos.ptr);
    a.cos_t = rope_cos();
    a.sin_t = rope_sin();
    check_hip(launch_backward(a, stream(), &timer_), "attention backward launch");
  }

  // The same backward with every buffer beyond the caller's tensors taken
  // from the device's fixed scratch array (noalloc_bwd_workspace): no device
  // memory is allocated, and nothing on the host either once the call's
  // sequence layout and RoPE table are resident.  No kernel timing.
  void LaunchAttnTrainBwdNoAlloc(const ShapeArgs& s, const void* d_out, const void* q_rot,
                                 const void* k_rot, const void* v, const void* out,
                                 const float* lse, void* dq, void* dk, void* dv) {
    if (s.total_tokens == 0) return;
    void* base = noalloc_scratch(device_);
    if (base == nullptr) {
      const hipError_t e = noalloc_scratch_init(device_);
      if (e != hipSuccess) {
        (void)hipGetLastError();
        fail(GLACIER_ATTN_ERR_DEVICE,
             std::string("the allocation-free backward's scratch is unavailable on this device: ") +
                 hipGetErrorString(e));
      }
      base = noalloc_scratch(device_);
    }
    int wide_tiles = 0;
    for (int b = 0; b < s.n_seqs; ++b)
      wide_tiles += (s.seq_start(b + 1) - s.seq_start(b) + kWideTile - 1) / kWideTile;
    const bool head_pairs = head_pairs_for(s.n_heads_q, s.n_heads_kv, s.head_dim, wide_tiles);
    NoAllocBwd w = noalloc_bwd_workspace(device_, base, s, n_cu_, split_ok_, head_pairs);
    BwdLaunch a = bwd_launch_of(BwdCall{s.total_tokens, s.n_heads_q, s.n_heads_kv, s.head_dim,
                                        s.precision, s.io_bf16, s.n_seqs == 1, w.n_tiles,
                                        w.pairs});
    a.dkdv_head_pairs = head_pairs;
    a.d_out = d_out; a.q_rot = q_rot; a.k_rot = k_rot; a.v = v; a.out = out;
    a.lse = lse; a.dq = dq; a.dk = dk; a.dv = dv;
    a.wk = w.wk;
    a.wv = w.wv;
    a.stats = w.stats;
    a.tiles_bwd = w.tiles_bwd;
    a.split = w.split;
    a.n_split_entries = w.n_split_entries;
    a.tiles_split = w.tiles_split;
    a.wk2 = w.wk2;
    a.wv2 = w.wv2;
    a.tiles_wide = w.tiles_wide;
    a.n_wide_entries = w.n_wide_entries;
    a.pos_of = w.pos_of;
    a.cos_t = w.cos_t;
    a.sin_t = w.sin_t;
    check_hip(launch_backward(a, stream(), nullptr), "attention backward launch");
  }

  // ---- projection with LoRA adapters (glacier_qkv.h) --------------------
  // GpuLoraEngine.ForwardQKV (GpuLoraEngine.Forward.cs:205-245) with the
  // LoRA deltas added on the device instead of AddLoraDeltaHost (:366-399).
  void ProjForward(ProjLaunch& a) {
    if (a.T == 0) return;
    ProjScratch(a, false);
    check_hip(launch_proj_forward(a, stream()), "projection forward launch");
  }

  // The block's LoraAdapter.Backward calls (LoraAdapter.cs:190-247).
  void ProjBackward(ProjLaunch& a) {
    if (a.T == 0) return;
    ProjScratch(a, true);
    check_hip(launch_proj_backward(a, stream()), "projection backward launch");
  }

  // ---- residual add and RMSNorm (glacier_norm.h) ------------------------
  // ElementwiseKernels.RMSNorm and TensorOps.Add (TransformerBlock.cs:318,
  // :505-506, :524, :579).
  void NormForward(const NormFwd& a) {
    if (a.rows == 0) return;
    check_hip(launch_rmsnorm_forward(a, stream(), &timer_), "rmsnorm forward launch");
  }

  // ElementwiseKernels.RMSNormBackward and the residual adds
  // (TransformerBlock.cs:672-677, :827-836).
  void NormBackward(NormBwd a) {
    if (a.rows == 0) return;
    a.dy_w = a.dy;
    if (a.d_weight != nullptr) {
      a.rstd = static_cast<float*>(rstd_.ensure(sizeof(float) * a.rows, "norm row scales"));
      // The weight gradient is formed after dx is stored; when dx overwrites
      // dy it reads a copy of dy taken first.
      if (a.dx == a.dy) {
        const size_t bytes = (size_t)a.rows * a.n * (a.io_bf16 ? 2 : 4);
        void* copy = dyw_.ensure(bytes, "norm dy copy");
        check_hip(hipMemcpyAsync(copy, a.dy, bytes, hipMemcpyDeviceToDevice, stream()),
                  "copy dy for the weight gradient");
        a.dy_w = copy;
      }
    }
    check_hip(launch_rmsnorm_backward(a, stream(), &timer_), "rmsnorm backward launch");
  }

  // ---- LM-head cross-entropy (glacier_lmhead.h) -------------------------
  // FusedCrossEntropyLoss.ComputeLoss / ComputeLossAndGradients
  // (FusedCrossEntropyLoss.cs:38-364): the kept rows are found on the host
  // from the host targets (:53, :190), as in the reference; the loss comes
  // back as one float.  Synchronises the stream.
  void LmHead(LmHeadLaunch a, const int32_t* targets, float* loss, int32_t* n_valid) {
    std::vector<int> rows, tgts, src_of;
    lmhead_rows(targets, a.T, a.V, rows, tgts, src_of);
    const int n = static_cast<int>(rows.size());
    if (n_valid != nullptr) *n_valid = n;
    *loss = 0.0f;
    if (a.T == 0 || (n == 0 && a.d_hidden == nullptr)) return;
    lmhead_shape(a, n);
    const LmHeadScratch need = lmhead_scratch(a);
    int* idx = static_cast<int*>(lm_idx_.ensure(need.idx, "LM-head row indices"));
    hipStream_t st = stream();
    if (n > 0) {
      check_hip(hipMemcpyAsync(idx, rows.data(), n * sizeof(int), hipMemcpyHostToDevice, st),
                "copy row indices");
      check_hip(hipMemcpyAsync(idx + n, tgts.data(), n * sizeof(int), hipMemcpyHostToDevice, st),
                "copy targets");
    }
    check_hip(hipMemcpyAsync(idx + 2 * n, src_of.data(), a.T * sizeof(int), hipMemcpyHostToDevice, st),
              "copy row map");
    a.rows = idx;
    a.targets = idx + n;
    a.src_of = idx + 2 * n;
    if (n > 0) {
      a.hv = lm_hv_.ensure(need.hv, "LM-head packed rows");
      a.logits = static_cast<float*>(lm_logits_.ensure(need.logits, "LM-head logits"));
      a.dl = a.io_bf16 ? lm_dl_.ensure(need.dl, "LM-head dlogits") : static_cast<void*>(a.logits);
      if (a.d_hidden != nullptr)
        a.dhv = static_cast<float*>(lm_dhv_.ensure(need.dhv, "LM-head packed gradient"));
      a.row_loss = static_cast<float*>(lm_loss_.ensure(need.row_loss, "LM-head losses"));
      a.loss = a.row_loss + n;
    }
    check_hip(launch_lmhead(a, st, blas()), "LM-head launch");
    float host_loss = 0.0f;
    if (n > 0)
      check_hip(hipMemcpyAsync(&host_loss, a.loss, sizeof(float), hipMemcpyDeviceToHost, st),
                "copy loss to host");
    check_hip(hipStreamSynchronize(st), "LM-head synchronize");
    *loss = host_loss;
  }

  // ---- host entry points (fp32 host tensors) ----------------------------
  // GpuLoraEngine.ForwardAttention (GpuLoraEngine.Forward.cs:467-512).
  void ForwardAttention(int /*layerIndex*/, float* q, float* k, const float* v,
                        float* attnOut, float* attnLse, const Shape& s) {
    if (s.total_tokens == 0) return;
    const size_t qb = (size_t)s.total_tokens * s.n_heads_q * s.head_dim * sizeof(float);
    const size_t kb = (size_t)s.total_tokens * s.n_heads_kv * s.head_dim * sizeof(float);
    const size_t lb = (size_t)s.n_heads_q * s.total_tokens * sizeof(float);
    EnsureAttnCapacity(s);
    hipStream_t st = stream();
    check_hip(hipMemcpyAsync(h_q_.ptr, q, qb, hipMemcpyHostToDevice, st), "copy q to device");
    check_hip(hipMemcpyAsync(h_k_.ptr, k, kb, hipMemcpyHostToDevice, st), "copy k to device");
    check_hip(hipMemcpyAsync(h_v_.ptr, v, kb, hipMemcpyHostToDevice, st), "copy v to device");
    const bool save = attnLse != nullptr;
    LaunchAttnTrainFwd(s, h_q_.ptr, h_k_.ptr, h_v_.ptr, h_out_.ptr,
                       save ? static_cast<float*>(h_lse_.ptr) : nullptr,
                       save ? h_qr_.ptr : nullptr, save ? h_kr_.ptr : nullptr);
    check_hip(hipMemcpyAsync(attnOut, h_out_.ptr, qb, hipMemcpyDeviceToHost, st), "copy out to host");
    if (save) {
      check_hip(hipMemcpyAsync(attnLse, h_lse_.ptr, lb, hipMemcpyDeviceToHost, st), "copy lse to host");
      check_hip(hipMemcpyAsync(q, h_qr_.ptr, qb, hipMemcpyDeviceToHost, st), "copy q_rot to host");
      check_hip(hipMemcpyAsync(k, h_kr_.ptr, kb, hipMemcpyDeviceToHost, st), "copy k_rot to host");
    }
    check_hip(hipStreamSynchronize(st), "forward attention");
  }

  // GpuLoraEngine.BackwardAttention (GpuLoraEngine.Backward.cs:414-458).
  void BackwardAttention(int /*layerIndex*/, const float* dAttnOut, const float* q,
                         const float* k, const float* v, const float* attnOut,
                         const float* attnLse, float* dq, float* dk, float* dv,
                         const Shape& s) {
    if (s.total_tokens == 0) return;
    const size_t qb = (size_t)s.total_tokens * s.n_heads_q * s.head_dim * sizeof(float);
    const size_t kb = (size_t)s.total_tokens * s.n_heads_kv * s.head_dim * sizeof(float);
    const size_t lb = (size_t)s.n_heads_q * s.total_tokens * sizeof(float);
    EnsureAttnCapacity(s);
    hipStream_t st = stream();
    check_hip(hipMemcpyAsync(h_dout_.ptr, dAttnOut, qb, hipMemcpyHostToDevice, st), "copy dO to device");
    check_hip(hipMemcpyAsync(h_q_.ptr, q, qb, hipMemcpyHostToDevice, st), "copy q to device");
    check_hip(hipMemcpyAsync(h_k_.ptr, k, kb, hipMemcpyHostToDevice, st), "copy k to device");
    check_hip(hipMemcpyAsync(h_v_.ptr, v, kb, hipMemcpyHostToDevice, st), "copy v to device");
    check_hip(hipMemcpyAsync(h_out_.ptr, attnOut, qb, hipMemcpyHostToDevice, st), "copy out to device");
    check_hip(hipMemcpyAsync(h_lse_.ptr, attnLse, lb, hipMemcpyHostToDevice, st), "copy lse to device");
    LaunchAttnTrainBwd(s, h_dout_.ptr, h_q_.ptr, h_k_.ptr, h_v_.ptr, h_out_.ptr,
                       static_cast<const float*>(h_lse_.ptr), h_dq_.ptr, h_dk_.ptr, h_dv_.ptr);
    check_hip(hipMemcpyAsync(dq, h_dq_.ptr, qb, hipMemcpyDeviceToHost, st), "copy dq to host");
    check_hip(hipMemcpyAsync(dk, h_dk_.ptr, kb, hipMemcpyDeviceToHost, st), "copy dk to host");
    check_hip(hipMemcpyAsync(dv, h_dv_.ptr, kb, hipMemcpyDeviceToHost, st), "copy dv to host");
    check_hip(hipStreamSynchronize(st), "backward attention");
  }

 private:
  // Device copies of the host tensors (GpuLoraEngine.Memory.cs:60-114).
  void EnsureAttnCapacity(const Shape& s) {
    const size_t qb = (size_t)s.total_tokens * s.n_heads_q * s.head_dim * sizeof(float);
    const size_t kb = (size_t)s.total_tokens * s.n_heads_kv * s.head_dim * sizeof(float);
    const size_t lb = (size_t)s.n_heads_q * s.total_tokens * sizeof(float);
    h_q_.ensure(qb, "q"); h_qr_.ensure(qb, "q_rot"); h_out_.ensure(qb, "attn_out");
    h_dout_.ensure(qb, "d_attn_out"); h_dq_.ensure(qb, "dq");
    h_k_.ensure(kb, "k"); h_kr_.ensure(kb, "k_rot"); h_v_.ensure(kb, "v");
    h_dk_.ensure(kb, "dk"); h_dv_.ensure(kb, "dv");
    h_lse_.ensure(lb, "lse");
  }

  // cos/sin per (position, pair) computed on the host with exactly the fp32
  // operations of RoPEKernel.cs:64-68 (glibc powf/cosf/sinf), uploaded once
  // per (length capacity, head_dim, theta).  One allocation holds the cosine
  // table and then the sine table (the bf16 forward takes the second as an
  // offset from the first).
  // real_dim: the call's own head size when head_dim is its padded one (the
  // angles are those of real_dim, in its first real_dim / 2 columns; the
  // padded columns rotate by the identity).
  void EnsureRopeTable(int max_len, int head_dim, float base, int real_dim) {
    if (max_len <= rope_len_ && head_dim == rope_dim_ && real_dim == rope_real_ && base == rope_base_)
      return;
    const int len = std::max(max_len, std::min(2 * rope_len_, GLACIER_ATTN_MAX_SEQ_LEN));
    const int half = head_dim / 2, rhalf = real_dim / 2;
    std::vector<float> cs((size_t)len * half, 1.0f), sn((size_t)len * half, 0.0f);
    std::vector<float> freq(rhalf);
    for (int i = 0; i < rhalf; i++) freq[i] = rope_freq(i, real_dim, base);
    for (int pos = 0; pos < len; pos++)
      for (int i = 0; i < rhalf; i++) {
        const float theta = static_cast<float>(pos) * freq[i];
        cs[(size_t)pos * half + i] = cosf(theta);
        sn[(size_t)pos * half + i] = sinf(theta);
      }
    const size_t bytes = cs.size() * sizeof(float);
    rope_.ensure(2 * bytes, "rope tables");
    check_hip(hipStreamSynchronize(stream()), "rope table");
    check_hip(hipMemcpy(rope_.ptr, cs.data(), bytes, hipMemcpyHostToDevice), "rope cos upload");
    check_hip(hipMemcpy(static_cast<char*>(rope_.ptr) + bytes, sn.data(), bytes, hipMemcpyHostToDevice),
              "rope sin upload");
    rope_len_ = len;
    rope_dim_ = head_dim;
    rope_real_ = real_dim;
    rope_base_ = base;
  }

  const TileSet& tiles_for(const Shape& s) {
    auto it = tile_cache_.find(s.cu);
    if (it != tile_cache_.end()) return *it->second;
    auto ts = std::make_unique<TileSet>();
    std::vector<TileDesc> nat;
    std::vector<int32_t> pos(s.total_tokens);
    const int n = static_cast<int>(s.cu.size()) - 1;
    for (int b = 0; b < n; ++b) {
      const int tok0 = s.cu[b], len = s.cu[b + 1] - s.cu[b];
      if (len <= 0) continue;
      const int nt = (len + kTile - 1) / kTile;
      for (int t = 0; t < nt; ++t) nat.push_back(TileDesc{tok0, len, t, 0});
      for (int i = 0; i < len; ++i) pos[tok0 + i] = i;
      ts->max_len = std::max(ts->max_len, len);
      ts->pairs += static_cast<long long>(len) * (len + 1) / 2;
    }
    ts->n_tiles = static_cast<int>(nat.size());
    if (ts->n_tiles > 65535)
      fail(GLACIER_ATTN_ERR_UNSUPPORTED, "more than 65535 tiles of 64 tokens in one call");
    // Longest query tiles first (they see the most keys), and key tiles with
    // the most query tiles first, so the long workgroups start earliest.
    std::vector<TileDesc> fwd = nat, kv = nat;
    std::stable_sort(fwd.begin(), fwd.end(),
                     [](const TileDesc& x, const TileDesc& y) { return x.tile > y.tile; });
    auto remaining = [](const TileDesc& x) { return (x.len + kTile - 1) / kTile - x.tile; };
    std::stable_sort(kv.begin(), kv.end(), [&](const TileDesc& x, const TileDesc& y) {
      return remaining(x) > remaining(y);
    });
    // Backward: dK/dV and dQ tiles share one launch, longest expected first
    // (bwd_tile_cost); the split tables likewise, with dK/dV tiles 0 ..
    // split - 1 of every sequence in query halves.
    auto backward_table = [&](int split, std::vector<TileDesc>& all) {
      std::vector<std::pair<int, TileDesc>> bw;
      for (int b = 0; b < n; ++b) {
        const int tok0 = s.cu[b], len = s.cu[b + 1] - s.cu[b];
        if (len <= 0) continue;
        const int nt = (len + kTile - 1) / kTile;
        bwd_entries(nt, split, [&](int t, int kind) {
          bw.push_back({bwd_tile_cost(nt, t, kind), TileDesc{tok0, len, t, kind}});
        });
      }
      std::stable_sort(bw.begin(), bw.end(),
                       [](const std::pair<int, TileDesc>& x, const std::pair<int, TileDesc>& y) {
                         return x.first > y.first;
                       });
      for (const auto& e : bw) all.push_back(e.second);
      return static_cast<int>(bw.size());
    };
    for (int b = 0; b < n; ++b) ts->seq_tiles.push_back((std::max(s.cu[b + 1] - s.cu[b], 0) + kTile - 1) / kTile);
    std::vector<TileDesc> all;
    all.insert(all.end(), fwd.begin(), fwd.end());
    backward_table(0, all);
    // only a layout of fewer backward entries than CUs (and an eighth) can
    // ever be split
    if (2 * static_cast<long long>(ts->n_tiles) < n_cu_ + n_cu_ / 8) {
      for (int split = 1; split <= kBwdMaxSplit; ++split) {
        ts->split_at[split] = static_cast<int>(all.size());
        ts->split_entries[split] = backward_table(split, all);
      }
    }
    // the 128-row backward table: dK/dV tiles of 128 keys and dQ tiles of 128
    // queries, longest expected first (bwd_wide_cost)
    // (and the same over query-head pairs: each dQ tile twice)
    for (const bool head_pairs : {false, true}) {
      std::vector<std::pair<int, TileDesc>> bw;
      int wide_tiles = 0;
      for (int b = 0; b < n; ++b) {
        const int tok0 = s.cu[b], len = s.cu[b + 1] - s.cu[b];
        if (len <= 0) continue;
        const int nt = (len + kWideTile - 1) / kWideTile;
        wide_tiles += nt;
        for (int t = 0; t < nt; ++t)
          for (int kind : wide_kinds(head_pairs))
            bw.push_back({bwd_wide_cost(len, t, kind, head_pairs), TileDesc{tok0, len, t, kind}});
      }
      std::stable_sort(bw.begin(), bw.end(),
                       [](const std::pair<int, TileDesc>& x, const std::pair<int, TileDesc>& y) {
                         return x.first > y.first;
                       });
      (head_pairs ? ts->wide2_at : ts->wide_at) = static_cast<int>(all.size());
      (head_pairs ? ts->wide2_entries : ts->wide_entries) = static_cast<int>(bw.size());
      ts->wide_tiles = wide_tiles;
      for (const auto& e : bw) all.push_back(e.second);
    }
    ts->tiles.ensure(all.size() * sizeof(TileDesc), "tile table");
    ts->pos.ensure(pos.size() * sizeof(int32_t), "position table");
    check_hip(hipStreamSynchronize(stream()), "tile table");
    check_hip(hipMemcpy(ts->tiles.ptr, all.data(), all.size() * sizeof(TileDesc),
                        hipMemcpyHostToDevice), "tile table upload");
    check_hip(hipMemcpy(ts->pos.ptr, pos.data(), pos.size() * sizeof(int32_t),
                        hipMemcpyHostToDevice), "position table upload");
    if (tile_cache_.size() >= 64) tile_cache_.clear();
    auto& ref = *ts;
    tile_cache_[s.cu] = std::move(ts);
    return ref;
  }

  void* blas() {
    if (blas_ == nullptr) {
      blas_ = create_blas_handle();
      if (blas_ == nullptr) fail(GLACIER_ATTN_ERR_DEVICE, "hipblasLtCreate failed");
    }
    return blas_;
  }

  void ProjScratch(ProjLaunch& a, bool backward) {
    const ProjScratchNeed need = proj_scratch_need(a, backward);
    auto get = [](DeviceBuffer& buf, long floats, const char* what) {
      return floats > 0 ? static_cast<float*>(buf.ensure(floats * sizeof(float), what)) : nullptr;
    };
    a.yf = get(yf_, need.yf, "projection scratch");
    a.dxf = get(dxf_, need.dxf, "dX scratch");
    a.lowrank = get(lowrank_, need.lowrank, "low-rank scratch");
    a.part = get(part_, need.part, "low-rank split sums");
  }

  int device_;
  int precision_;
  hipStream_t own_stream_ = nullptr;
  hipStream_t user_stream_ = nullptr;
  bool has_user_stream_ = false;
  std::mutex mutex_;
  KernelTimer timer_;
  std::map<std::vector<int32_t>, std::unique_ptr<TileSet>> tile_cache_;
  DeviceBuffer rope_;  // [rope_len_][rope_dim_ / 2] cosines, then as many sines
  const float* rope_cos() const { return static_cast<const float*>(rope_.ptr); }
  const float* rope_sin() const { return rope_cos() + (size_t)rope_len_ * (rope_dim_ / 2); }
  int rope_len_ = 0, rope_dim_ = 0, rope_real_ = 0;
  float rope_base_ = 0.0f;
  // device-path scratch
  DeviceBuffer kc_, vc_, wk_, wv_, wk2_, wv2_, stats_;
  // padded copies for head sizes the kernels are not built for
  DeviceBuffer pad_q_, pad_k_, pad_v_, pad_o_, pad_qr_, pad_kr_, pad_do_, pad_dq_, pad_dk_, pad_dv_;
  int bwd_variant_ = kBwdAuto;
  int n_cu_ = 0;          // compute units of the device
  bool split_ok_ = true;  // dK/dV tiles may be split (GLACIER_ATTN_BWD_SPLIT)
  int fwd_rows_ = 0;      // bf16 forward rows per workgroup (GLACIER_ATTN_FWD_ROWS; 0: auto)
  int bwd_pairs_mode_ = -1;  // wide backward over head pairs: 1 on, 0 off, -1 auto (GLACIER_ATTN_BWD_PAIRS)
  // projection scratch and the hipBLASLt handle (created on first use)
  DeviceBuffer yf_, dxf_, lowrank_, part_;
  DeviceBuffer rstd_, dyw_;  // RMSNorm backward row scales, dy copy (weight gradient)
  DeviceBuffer lm_idx_, lm_hv_, lm_logits_, lm_dl_, lm_dhv_, lm_loss_;  // LM head
  void* blas_ = nullptr;
  // host-path device copies
  DeviceBuffer h_q_, h_k_, h_v_, h_out_, h_lse_, h_qr_, h_kr_, h_dout_, h_dq_, h_dk_, h_dv_;
};

namespace {

// Validates a shape before anything touches the GPU.  Throws Error.
// Validates one call's shape without copying anything (on success nothing
// is allocated); make_shape builds the engine's cached form from it.
ShapeArgs make_shape_args(int total_tokens, int n_seqs, const int32_t* cu, int hq, int hkv,
                          int d, float base, int precision, int io) {
  if (n_seqs < 1) fail(GLACIER_ATTN_ERR_INVALID_ARGUMENT, "n_seqs must be >= 1");
  if (total_tokens < 0) fail(GLACIER_ATTN_ERR_INVALID_ARGUMENT, "total_tokens must be >= 0");
  if (hq <= 0 || hkv <= 0)
    fail(GLACIER_ATTN_ERR_INVALID_ARGUMENT, "head counts must be positive");
  if (hq % hkv != 0)
    fail(GLACIER_ATTN_ERR_INVALID_ARGUMENT,
         "n_heads_q (" + std::to_string(hq) + ") must be a multiple of n_heads_kv (" +
             std::to_string(hkv) + ")");
  if (d <= 0 || d > 1024)
    fail(GLACIER_ATTN_ERR_INVALID_ARGUMENT,
         "GPU training attention requires 1 <= headDim <= 1024, got " + std::to_string(d) + ".");
  if (!(base > 0.0f) || !std::isfinite(base))
    fail(GLACIER_ATTN_ERR_INVALID_ARGUMENT, "rope_freq_base must be positive and finite");
  if (precision != GLACIER_ATTN_PREC_FP32 && precision != GLACIER_ATTN_PREC_BF16)
    fail(GLACIER_ATTN_ERR_INVALID_ARGUMENT, "unknown precision " + std::to_string(precision));
  if (io != GLACIER_ATTN_IO_F32 && io != GLACIER_ATTN_IO_BF16)
    fail(GLACIER_ATTN_ERR_INVALID_ARGUMENT, "unknown io dtype " + std::to_string(io));
  if (io == GLACIER_ATTN_IO_BF16 && precision != GLACIER_ATTN_PREC_BF16)
    fail(GLACIER_ATTN_ERR_INVALID_ARGUMENT, "bf16 device tensors need GLACIER_ATTN_PREC_BF16");
  if (cu == nullptr) {
    if (n_seqs != 1)
      fail(GLACIER_ATTN_ERR_INVALID_ARGUMENT, "cu_seqlens is required when n_seqs > 1");
  } else {
    if (cu[0] != 0) fail(GLACIER_ATTN_ERR_INVALID_ARGUMENT, "cu_seqlens[0] must be 0");
    for (int b = 1; b <= n_seqs; ++b)
      if (cu[b] < cu[b - 1])
        fail(GLACIER_ATTN_ERR_INVALID_ARGUMENT, "cu_seqlens must be non-decreasing");
    if (cu[n_seqs] != total_tokens)
      fail(GLACIER_ATTN_ERR_INVALID_ARGUMENT, "cu_seqlens[n_seqs] must equal total_tokens");
  }
  ShapeArgs s;
  s.total_tokens = total_tokens;
  s.n_seqs = n_seqs;
  s.cu = cu;
  for (int b = 0; b < n_seqs; ++b) s.max_len = std::max(s.max_len, s.seq_start(b + 1) - s.seq_start(b));
  if (!GpuAttentionEngine::SupportedHeadDim(d))
    fail(GLACIER_ATTN_ERR_UNSUPPORTED, "head_dim " + std::to_string(d) +
                                           " is not supported by the GPU kernels (1 to 256)");
  if (GpuAttentionEngine::PaddedHeadDim(d) > 128 && precision == GLACIER_ATTN_PREC_FP32)
    fail(GLACIER_ATTN_ERR_UNSUPPORTED,
         "head_dim " + std::to_string(d) + " runs in GLACIER_ATTN_PREC_BF16 only (its fp32 "
         "key/value tiles do not fit the LDS)");
  if (s.max_len > GLACIER_ATTN_MAX_SEQ_LEN)
    fail(GLACIER_ATTN_ERR_UNSUPPORTED, "sequence of " + std::to_string(s.max_len) +
                                           " tokens exceeds GLACIER_ATTN_MAX_SEQ_LEN");
  if ((long long)total_tokens * hq * d >= (1LL << 40))
    fail(GLACIER_ATTN_ERR_UNSUPPORTED, "tensor too large");
  s.n_heads_q = hq;
  s.n_heads_kv = hkv;
  s.head_dim = d;
  s.rope_freq_base = base;
  s.precision = precision;
  s.io_bf16 = io == GLACIER_ATTN_IO_BF16;
  return s;
}

Shape make_shape(int total_tokens, int n_seqs, const int32_t* cu, int hq, int hkv,
                 int d, float base, int precision, int io) {
  const ShapeArgs a = make_shape_args(total_tokens, n_seqs, cu, hq, hkv, d, base, precision, io);
  Shape s;
  s.cu.resize(n_seqs + 1);
  for (int b = 0; b <= n_seqs; ++b) s.cu[b] = a.seq_start(b);
  s.total_tokens = a.total_tokens;
  s.n_heads_q = a.n_heads_q;
  s.n_heads_kv = a.n_heads_kv;
  s.head_dim = a.head_dim;
  s.rope_freq_base = a.rope_freq_base;
  s.precision = a.precision;
  s.io_bf16 = a.io_bf16;
  return s;
}

Shape shape_of(const glacier_attn_desc* desc) {
  if (desc == nullptr) fail(GLACIER_ATTN_ERR_INVALID_ARGUMENT, "desc is NULL");
  return make_shape(desc->total_tokens, desc->n_seqs, desc->cu_seqlens, desc->n_heads_q,
                    desc->n_heads_kv, desc->head_dim, desc->rope_freq_base,
                    desc->precision, desc->io_dtype);
}

// Validates a projection call and fills the launch (pointers only).
bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

ProjLaunch proj_launch_of(const glacier_proj_desc* desc, const void* x, const glacier_lora_proj* proj,
                          int n_proj, bool backward) {
  if (desc == nullptr) fail(GLACIER_ATTN_ERR_INVALID_ARGUMENT, "desc is NULL");
  const glacier_proj_desc& d = *desc;
  if (d.total_tokens < 0) fail(GLACIER_ATTN_ERR_INVALID_ARGUMENT, "total_tokens must be >= 0");
  if (d.in_features <= 0) fail(GLACIER_ATTN_ERR_INVALID_ARGUMENT, "in_features must be positive");
  if (d.precision != GLACIER_ATTN_PREC_FP32 && d.precision != GLACIER_ATTN_PREC_BF16)
    fail(GLACIER_ATTN_ERR_INVALID_ARGUMENT, "unknown precision " + std::to_string(d.precision));
  if (d.io_dtype != GLACIER_ATTN_IO_F32 && d.io_dtype != GLACIER_ATTN_IO_BF16)
    fail(GLACIER_ATTN_ERR_INVALID_ARGUMENT, "unknown io dtype " + std::to_string(d.io_dtype));
  if (d.io_dtype == GLACIER_ATTN_IO_BF16 && d.precision != GLACIER_ATTN_PREC_BF16)
    fail(GLACIER_ATTN_ERR_INVALID_ARGUMENT, "bf16 device tensors need GLACIER_ATTN_PREC_BF16");
  if (proj == nullptr) fail(GLACIER_ATTN_ERR_INVALID_ARGUMENT, "proj is NULL");
  if (n_proj < 1 || n_proj > GLACIER_PROJ_MAX_PROJ)
    fail(GLACIER_ATTN_ERR_INVALID_ARGUMENT, "n_proj must be 1.." + std::to_string(GLACIER_PROJ_MAX_PROJ));
  if (d.total_tokens > 0 && x == nullptr) fail(GLACIER_ATTN_ERR_INVALID_ARGUMENT, "x is NULL");
  ProjLaunch a{};
  a.T = d.total_tokens;
  a.in = d.in_features;
  a.rank = d.rank;
  a.io_bf16 = d.io_dtype == GLACIER_ATTN_IO_BF16;
  a.n_proj = n_proj;
  a.x = x;
  bool any_lora = false;
  for (int p = 0; p < n_proj; ++p) {
    const glacier_lora_proj& g = proj[p];
    const std::string at = "proj[" + std::to_string(p) + "]";
    if (g.out_features <= 0) fail(GLACIER_ATTN_ERR_INVALID_ARGUMENT, at + ".out_features must be positive");
    if (d.total_tokens > 0) {
      if (g.w == nullptr) fail(GLACIER_ATTN_ERR_INVALID_ARGUMENT, at + ".w is NULL");
      if (!backward && g.y == nullptr) fail(GLACIER_ATTN_ERR_INVALID_ARGUMENT, at + ".y is NULL");
      if (backward && g.dy == nullptr) fail(GLACIER_ATTN_ERR_INVALID_ARGUMENT, at + ".dy is NULL");
    }
    if (g.lora_a != nullptr) {
      any_lora = true;
      if (g.lora_b == nullptr) fail(GLACIER_ATTN_ERR_INVALID_ARGUMENT, at + ".lora_b is NULL");
      if (!std::isfinite(g.scaling)) fail(GLACIER_ATTN_ERR_INVALID_ARGUMENT, at + ".scaling is not finite");
    }
    a.p[p] = ProjSpec{g.w, g.bias, g.lora_a, g.lora_b, g.scaling, g.out_features,
                      g.y, g.dy, g.grad_a, g.grad_b};
  }
  if (any_lora && (d.rank < 1 || d.rank > GLACIER_PROJ_MAX_RANK))
    fail(GLACIER_ATTN_ERR_INVALID_ARGUMENT,
         "rank must be 1.." + std::to_string(GLACIER_PROJ_MAX_RANK) + " when an adapter is given");
  if (d.in_features % 4 != 0)
    fail(GLACIER_ATTN_ERR_UNSUPPORTED, "in_features must be a multiple of 4");
  for (int p = 0; p < n_proj; ++p)
    if (proj[p].out_features % 4 != 0)
      fail(GLACIER_ATTN_ERR_UNSUPPORTED, "out_features must be a multiple of 4");
  // the kernels move 4 consecutive elements of x, y, dy, dx and the adapters at once
  if (!aligned16(x)) fail(GLACIER_ATTN_ERR_UNSUPPORTED, "x must be 16-byte aligned");
  for (int p = 0; p < n_proj; ++p)
    if (!aligned16(backward ? proj[p].dy : proj[p].y) || !aligned16(proj[p].lora_a) ||
        !aligned16(proj[p].lora_b))
      fail(GLACIER_ATTN_ERR_UNSUPPORTED,
           "proj[" + std::to_string(p) + "]." + (backward ? "dy" : "y") +
               ", .lora_a and .lora_b must be 16-byte aligned");
  if ((long long)d.total_tokens * std::max(d.in_features, 1) >= (1LL << 31))
    fail(GLACIER_ATTN_ERR_UNSUPPORTED, "tensor too large");
  for (int p = 0; p < n_proj; ++p)
    if ((long long)d.total_tokens * proj[p].out_features >= (1LL << 31) ||
        (long long)proj[p].out_features * d.in_features >= (1LL << 31))
      fail(GLACIER_ATTN_ERR_UNSUPPORTED, "tensor too large");
  return a;
}

// Checks a glacier_norm_desc before any device work.
void norm_check(const glacier_norm_desc* desc) {
  if (desc == nullptr) fail(GLACIER_ATTN_ERR_INVALID_ARGUMENT, "desc is NULL");
  const glacier_norm_desc& d = *desc;
  if (d.rows < 0) fail(GLACIER_ATTN_ERR_INVALID_ARGUMENT, "rows must be >= 0");
  if (d.n <= 0) fail(GLACIER_ATTN_ERR_INVALID_ARGUMENT, "n must be positive");
  if (d.io_dtype != GLACIER_ATTN_IO_F32 && d.io_dtype != GLACIER_ATTN_IO_BF16)
    fail(GLACIER_ATTN_ERR_INVALID_ARGUMENT, "unknown io dtype " + std::to_string(d.io_dtype));
  if (!std::isfinite(d.eps) || d.eps < 0.0f)
    fail(GLACIER_ATTN_ERR_INVALID_ARGUMENT, "eps must be finite and >= 0");
  if (d.n % 4 != 0) fail(GLACIER_ATTN_ERR_UNSUPPORTED, "n must be a multiple of 4");
  if (d.n > GLACIER_NORM_MAX_N)
    fail(GLACIER_ATTN_ERR_UNSUPPORTED, "n must be at most " + std::to_string(GLACIER_NORM_MAX_N));
  if ((long long)d.rows * d.n >= (1LL << 31)) fail(GLACIER_ATTN_ERR_UNSUPPORTED, "tensor too large");
}

// Non-null (when the call has rows) and 16-byte aligned: the kernels move 4
// consecutive elements at once.
void need_row_tensor(const void* p, const char* name, bool has_rows) {
  if (has_rows && p == nullptr) fail(GLACIER_ATTN_ERR_INVALID_ARGUMENT, std::string(name) + " is NULL");
  if (!aligned16(p)) fail(GLACIER_ATTN_ERR_UNSUPPORTED, std::string(name) + " must be 16-byte aligned");
}

void need(const void* p, const char* name) {
  if (p == nullptr) fail(GLACIER_ATTN_ERR_INVALID_ARGUMENT, std::string(name) + " is NULL");
}

template <typename F>
int guarded(F&& f) {
  try {
    f();
    g_last_error.clear();
    return GLACIER_ATTN_OK;
  } catch (const Error& e) {
    g_last_error = e.what();
    return e.code();
  } catch (const std::bad_alloc&) {
    g_last_error = "host allocation failed";
    return GLACIER_ATTN_ERR_OUT_OF_MEMORY;
  } catch (const std::exception& e) {
    g_last_error = e.what();
    return GLACIER_ATTN_ERR_DEVICE;
  }
}

const char* const kKernelNames[kKernCount] = {
    "rope_k", "attn_fwd", "attn_bwd", "attn_bwd_reduce", "rmsnorm_fwd", "rmsnorm_bwd",
    "attn_bwd_stats",
};

}  // namespace
}  // namespace glacier

struct glacier_attn_ctx {
  std::unique_ptr<glacier::GpuAttentionEngine> eng;
};

using glacier::fail;
using glacier::guarded;
using glacier::need;

extern "C" {

int glacier_attn_create(int device_ordinal, int precision, glacier_attn_ctx** out) {
  return guarded([&] {
    need(out, "out");
    *out = nullptr;
    if (precision != GLACIER_ATTN_PREC_FP32 && precision != GLACIER_ATTN_PREC_BF16)
      fail(GLACIER_ATTN_ERR_INVALID_ARGUMENT, "unknown precision " + std::to_string(precision));
    auto ctx = std::make_unique<glacier_attn_ctx>();
    ctx->eng = std::make_unique<glacier::GpuAttentionEngine>(device_ordinal, precision);
    *out = ctx.release();
  });
}

void glacier_attn_destroy(glacier_attn_ctx* ctx) { delete ctx; }

const char* glacier_attn_last_error(void) { return glacier::g_last_error.c_str(); }

int glacier_attn_supports(int seq_len, int head_dim) {
  return glacier::GpuAttentionEngine::SupportsAttention(seq_len, head_dim) ? 1 : 0;
}

int glacier_attn_forward_host(glacier_attn_ctx* ctx, int layer_index, float* q, float* k,
                              const float* v, float* attn_out, float* attn_lse, int seq_len,
                              int n_heads_q, int n_heads_kv, int head_dim,
                              float rope_freq_base) {
  return guarded([&] {
    const int prec = ctx != nullptr ? ctx->eng->precision() : GLACIER_ATTN_PREC_FP32;
    glacier::Shape s = glacier::make_shape(seq_len, 1, nullptr, n_heads_q, n_heads_kv, head_dim,
                                           rope_freq_base, prec, GLACIER_ATTN_IO_F32);
    need(ctx, "ctx");
    need(q, "q"); need(k, "k"); need(v, "v"); need(attn_out, "attn_out");
    std::lock_guard<std::mutex> g(ctx->eng->lock());
    ctx->eng->activate();
    ctx->eng->ForwardAttention(layer_index, q, k, v, attn_out, attn_lse, s);
  });
}

int glacier_attn_backward_host(glacier_attn_ctx* ctx, int layer_index, const float* d_attn_out,
                               const float* q, const float* k, const float* v,
                               const float* attn_out, const float* attn_lse, float* dq,
                               float* dk, float* dv, int seq_len, int n_heads_q,
                               int n_heads_kv, int head_dim, float rope_freq_base) {
  return guarded([&] {
    const int prec = ctx != nullptr ? ctx->eng->precision() : GLACIER_ATTN_PREC_FP32;
    glacier::Shape s = glacier::make_shape(seq_len, 1, nullptr, n_heads_q, n_heads_kv, head_dim,
                                           rope_freq_base, prec, GLACIER_ATTN_IO_F32);
    need(ctx, "ctx");
    need(d_attn_out, "d_attn_out"); need(q, "q"); need(k, "k"); need(v, "v");
    need(attn_out, "attn_out"); need(attn_lse, "attn_lse");
    need(dq, "dq"); need(dk, "dk"); need(dv, "dv");
    std::lock_guard<std::mutex> g(ctx->eng->lock());
    ctx->eng->activate();
    ctx->eng->BackwardAttention(layer_index, d_attn_out, q, k, v, attn_out, attn_lse, dq, dk, dv,
                                s);
  });
}

int glacier_attn_forward(glacier_attn_ctx* ctx, const glacier_attn_desc* desc, const void* q,
                         const void* k, const void* v, void* out, float* lse, void* q_rot,
                         void* k_rot) {
  return guarded([&] {
    glacier::Shape s = glacier::shape_of(desc);
    need(ctx, "ctx");
    if (s.total_tokens > 0) {
      need(q, "q"); need(k, "k"); need(v, "v"); need(out, "out");
    }
    std::lock_guard<std::mutex> g(ctx->eng->lock());
    ctx->eng->activate();
    ctx->eng->LaunchAttnTrainFwd(s, q, k, v, out, lse, q_rot, k_rot);
  });
}

int glacier_attn_backward(glacier_attn_ctx* ctx, const glacier_attn_desc* desc,
                          const void* d_out, const void* q_rot, const void* k_rot, const void* v,
                          const void* out, const float* lse, void* dq, void* dk, void* dv) {
  return guarded([&] {
    glacier::Shape s = glacier::shape_of(desc);
    need(ctx, "ctx");
    if (s.total_tokens > 0) {
      need(d_out, "d_out"); need(q_rot, "q_rot"); need(k_rot, "k_rot"); need(v, "v");
      need(out, "out"); need(lse, "lse"); need(dq, "dq"); need(dk, "dk"); need(dv, "dv");
    }
    std::lock_guard<std::mutex> g(ctx->eng->lock());
    ctx->eng->activate();
    ctx->eng->LaunchAttnTrainBwd(s, d_out, q_rot, k_rot, v, out, lse, dq, dk, dv);
  });
}

int glacier_attn_backward_noalloc(glacier_attn_ctx* ctx, const glacier_attn_desc* desc,
                                  const void* d_out, const void* q_rot, const void* k_rot,
                                  const void* v, const void* out, const float* lse, void* dq,
                                  void* dk, void* dv) {
  return guarded([&] {
    if (desc == nullptr) glacier::fail(GLACIER_ATTN_ERR_INVALID_ARGUMENT, "desc is NULL");
    const glacier::ShapeArgs s = glacier::make_shape_args(
        desc->total_tokens, desc->n_seqs, desc->cu_seqlens, desc->n_heads_q, desc->n_heads_kv,
        desc->head_dim, desc->rope_freq_base, desc->precision, desc->io_dtype);
    if (glacier::GpuAttentionEngine::PaddedHeadDim(s.head_dim) != s.head_dim)
      glacier::fail(GLACIER_ATTN_ERR_UNSUPPORTED,
                    "the allocation-free backward takes head sizes 32, 64, 96, 128 and 256, not " +
                        std::to_string(s.head_dim) + " (other sizes need padded copies)");
    need(ctx, "ctx");
    if (s.total_tokens > 0) {
      need(d_out, "d_out"); need(q_rot, "q_rot"); need(k_rot, "k_rot"); need(v, "v");
      need(out, "out"); need(lse, "lse"); need(dq, "dq"); need(dk, "dk"); need(dv, "dv");
    }
    std::lock_guard<std::mutex> g(ctx->eng->lock());
    ctx->eng->activate();
    ctx->eng->LaunchAttnTrainBwdNoAlloc(s, d_out, q_rot, k_rot, v, out, lse, dq, dk, dv);
  });
}

int glacier_attn_set_stream(glacier_attn_ctx* ctx, void* hip_stream) {
  return guarded([&] {
    need(ctx, "ctx");
    std::lock_guard<std::mutex> g(ctx->eng->lock());
    ctx->eng->set_stream(static_cast<hipStream_t>(hip_stream));
  });
}

int glacier_attn_use_own_stream(glacier_attn_ctx* ctx) {
  return guarded([&] {
    need(ctx, "ctx");
    std::lock_guard<std::mutex> g(ctx->eng->lock());
    ctx->eng->use_own_stream();
  });
}

int glacier_attn_synchronize(glacier_attn_ctx* ctx) {
  return guarded([&] {
    need(ctx, "ctx");
    std::lock_guard<std::mutex> g(ctx->eng->lock());
    ctx->eng->activate();
    glacier::check_hip(hipStreamSynchronize(ctx->eng->stream()), "synchronize");
  });
}

int glacier_attn_set_kernel_timing(glacier_attn_ctx* ctx, int enable) {
  return guarded([&] {
    need(ctx, "ctx");
    std::lock_guard<std::mutex> g(ctx->eng->lock());
    ctx->eng->activate();
    glacier::check_hip(hipStreamSynchronize(ctx->eng->stream()), "synchronize");
    ctx->eng->timer().reset();
    ctx->eng->timer().enabled = enable != 0;
  });
}

int glacier_attn_kernel_count(void) { return glacier::kKernCount; }

const char* glacier_attn_kernel_name(int id) {
  if (id < 0 || id >= glacier::kKernCount) return nullptr;
  return glacier::kKernelNames[id];
}

int glacier_attn_kernel_time(glacier_attn_ctx* ctx, int id, double* total_ms, int64_t* launches) {
  return guarded([&] {
    need(ctx, "ctx");
    need(total_ms, "total_ms");
    need(launches, "launches");
    if (id < 0 || id >= glacier::kKernCount)
      fail(GLACIER_ATTN_ERR_INVALID_ARGUMENT, "kernel id out of range");
    std::lock_guard<std::mutex> g(ctx->eng->lock());
    ctx->eng->activate();
    glacier::check_hip(hipStreamSynchronize(ctx->eng->stream()), "synchronize");
    glacier::check_hip(ctx->eng->timer().collect(), "kernel timing");
    *total_ms = ctx->eng->timer().total_ms(id);
    *launches = ctx->eng->timer().launches(id);
  });
}

int glacier_proj_forward(glacier_attn_ctx* ctx, const glacier_proj_desc* desc, const void* x,
                         const glacier_lora_proj* proj, int n_proj) {
  return guarded([&] {
    glacier::ProjLaunch a = glacier::proj_launch_of(desc, x, proj, n_proj, false);
    need(ctx, "ctx");
    std::lock_guard<std::mutex> g(ctx->eng->lock());
    ctx->eng->activate();
    ctx->eng->ProjForward(a);
  });
}

int glacier_proj_backward(glacier_attn_ctx* ctx, const glacier_proj_desc* desc, const void* x,
                          const glacier_lora_proj* proj, int n_proj, void* dx) {
  return guarded([&] {
    glacier::ProjLaunch a = glacier::proj_launch_of(desc, x, proj, n_proj, true);
    need(ctx, "ctx");
    if (desc->total_tokens > 0) need(dx, "dx");
    if (!glacier::aligned16(dx)) glacier::fail(GLACIER_ATTN_ERR_UNSUPPORTED, "dx must be 16-byte aligned");
    a.dx = dx;
    std::lock_guard<std::mutex> g(ctx->eng->lock());
    ctx->eng->activate();
    ctx->eng->ProjBackward(a);
  });
}

int glacier_rmsnorm_forward(glacier_attn_ctx* ctx, const glacier_norm_desc* desc, const void* x,
                            const void* delta, const float* weight, void* x1, void* y) {
  return guarded([&] {
    glacier::norm_check(desc);
    const bool rows = desc->rows > 0;
    glacier::need_row_tensor(x, "x", rows);
    glacier::need_row_tensor(weight, "weight", rows);
    glacier::need_row_tensor(y, "y", rows);
    glacier::need_row_tensor(delta, "delta", false);
    if (delta != nullptr) glacier::need_row_tensor(x1, "x1 (required with delta)", rows);
    need(ctx, "ctx");
    glacier::NormFwd a{desc->rows, desc->n, desc->eps, desc->io_dtype == GLACIER_ATTN_IO_BF16,
                       x, delta, weight, delta != nullptr ? x1 : nullptr, y};
    std::lock_guard<std::mutex> g(ctx->eng->lock());
    ctx->eng->activate();
    ctx->eng->NormForward(a);
  });
}

int glacier_rmsnorm_backward(glacier_attn_ctx* ctx, const glacier_norm_desc* desc, const void* dy,
                             const void* x, const float* weight, const void* d_residual, void* dx,
                             float* d_weight) {
  return guarded([&] {
    glacier::norm_check(desc);
    const bool rows = desc->rows > 0;
    glacier::need_row_tensor(dy, "dy", rows);
    glacier::need_row_tensor(x, "x", rows);
    glacier::need_row_tensor(weight, "weight", rows);
    glacier::need_row_tensor(dx, "dx", rows);
    glacier::need_row_tensor(d_residual, "d_residual", false);
    glacier::need_row_tensor(d_weight, "d_weight", false);
    need(ctx, "ctx");
    glacier::NormBwd a{desc->rows, desc->n, desc->eps, desc->io_dtype == GLACIER_ATTN_IO_BF16,
                       dy, x, weight, d_residual, dx, d_weight, nullptr, dy};
    std::lock_guard<std::mutex> g(ctx->eng->lock());
    ctx->eng->activate();
    ctx->eng->NormBackward(a);
  });
}

namespace {

int lmhead_call(glacier_attn_ctx* ctx, const glacier_lmhead_desc* desc, const void* hidden,
                const int32_t* targets, const void* weight, void* d_hidden, float* loss,
                int32_t* n_valid, bool grad) {
  return guarded([&] {
    using glacier::fail;
    if (desc == nullptr) fail(GLACIER_ATTN_ERR_INVALID_ARGUMENT, "desc is NULL");
    const glacier_lmhead_desc& d = *desc;
    if (d.tokens < 0) fail(GLACIER_ATTN_ERR_INVALID_ARGUMENT, "tokens must be >= 0");
    if (d.hidden <= 0) fail(GLACIER_ATTN_ERR_INVALID_ARGUMENT, "hidden must be positive");
    if (d.vocab <= 0) fail(GLACIER_ATTN_ERR_INVALID_ARGUMENT, "vocab must be positive");
    if (d.precision != GLACIER_ATTN_PREC_FP32 && d.precision != GLACIER_ATTN_PREC_BF16)
      fail(GLACIER_ATTN_ERR_INVALID_ARGUMENT, "unknown precision " + std::to_string(d.precision));
    if (d.io_dtype != GLACIER_ATTN_IO_F32 && d.io_dtype != GLACIER_ATTN_IO_BF16)
      fail(GLACIER_ATTN_ERR_INVALID_ARGUMENT, "unknown io dtype " + std::to_string(d.io_dtype));
    if (d.io_dtype == GLACIER_ATTN_IO_BF16 && d.precision != GLACIER_ATTN_PREC_BF16)
      fail(GLACIER_ATTN_ERR_INVALID_ARGUMENT, "bf16 device tensors need GLACIER_ATTN_PREC_BF16");
    need(loss, "loss");
    const bool rows = d.tokens > 0;
    if (rows && targets == nullptr) fail(GLACIER_ATTN_ERR_INVALID_ARGUMENT, "targets is NULL");
    glacier::need_row_tensor(hidden, "hidden", rows);
    glacier::need_row_tensor(weight, "weight", rows);
    if (grad) glacier::need_row_tensor(d_hidden, "d_hidden", rows);
    if (d.hidden % 8 != 0) fail(GLACIER_ATTN_ERR_UNSUPPORTED, "hidden must be a multiple of 8");
    if ((long long)d.tokens * d.hidden >= (1LL << 31) || (long long)d.vocab * d.hidden >= (1LL << 31))
      fail(GLACIER_ATTN_ERR_UNSUPPORTED, "tensor too large");
    if ((long long)d.vocab + 8 >= (1LL << 31)) fail(GLACIER_ATTN_ERR_UNSUPPORTED, "vocab too large");
    need(ctx, "ctx");
    // Switched off: the first GPU run of this path (fp32, 32 x 896 hidden,
    // vocabulary 151936) ended in an illegal memory access, and no cause has
    // been shown yet; nothing is launched until one is.
    fail(GLACIER_ATTN_ERR_UNSUPPORTED,
         "the device LM-head path is switched off: its first GPU run faulted and the cause is not "
         "yet known");
    glacier::LmHeadLaunch a{};
    a.T = d.tokens;
    a.H = d.hidden;
    a.V = d.vocab;
    a.io_bf16 = d.io_dtype == GLACIER_ATTN_IO_BF16;
    a.hidden = hidden;
    a.weight = weight;
    a.d_hidden = grad ? d_hidden : nullptr;
    std::lock_guard<std::mutex> g(ctx->eng->lock());
    ctx->eng->activate();
    ctx->eng->LmHead(a, targets, loss, n_valid);
  });
}

}  // namespace

// ---- the 'LORA' v1 adapter file (glacier_lora_file.h) ---------------------
int glacier_lora_save(const char* path, int32_t layer_count, int32_t rank, float alpha,
                      int32_t n_tensors, const char* const* names, const int32_t* dim0,
                      const int32_t* dim1, const float* const* data) {
  return guarded([&] {
    std::string err;
    const int rc = glacier::lora::save(path, layer_count, rank, alpha, n_tensors, names, dim0, dim1,
                                       data, err);
    if (rc != GLACIER_ATTN_OK) glacier::fail(rc, err);
  });
}

int glacier_lora_open(const char* path, glacier_lora_header* header, glacier_lora_reader** reader) {
  return guarded([&] {
    std::string err;
    const int rc = glacier::lora::open(path, header, reader, err);
    if (rc != GLACIER_ATTN_OK) glacier::fail(rc, err);
  });
}

int glacier_lora_next(glacier_lora_reader* reader, char* name, int32_t name_cap, int32_t* dim0,
                      int32_t* dim1) {
  return guarded([&] {
    std::string err;
    const int rc = glacier::lora::next(reader, name, name_cap, dim0, dim1, err);
    if (rc != GLACIER_ATTN_OK) glacier::fail(rc, err);
  });
}

int glacier_lora_read(glacier_lora_reader* reader, float* dst, int32_t transpose) {
  return guarded([&] {
    std::string err;
    const int rc = glacier::lora::read(reader, dst, transpose, err);
    if (rc != GLACIER_ATTN_OK) glacier::fail(rc, err);
  });
}

void glacier_lora_close(glacier_lora_reader* reader) { glacier::lora::close(reader); }

int glacier_lmhead_loss(glacier_attn_ctx* ctx, const glacier_lmhead_desc* desc, const void* hidden,
                        const int32_t* targets, const void* weight, float* loss, int32_t* n_valid) {
  return lmhead_call(ctx, desc, hidden, targets, weight, nullptr, loss, n_valid, false);
}

int glacier_lmhead_loss_and_grad(glacier_attn_ctx* ctx, const glacier_lmhead_desc* desc,
                                 const void* hidden, const int32_t* targets, const void* weight,
                                 void* d_hidden, float* loss, int32_t* n_valid) {
  return lmhead_call(ctx, desc, hidden, targets, weight, d_hidden, loss, n_valid, true);
}

}  // extern "C"
