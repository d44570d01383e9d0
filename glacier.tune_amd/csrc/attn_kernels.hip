// attn_kernels.hip -- gfx950 kernels of the causal GQA attention path.
//
// Forward  (GpuLoraEngine.Forward.cs:401-465 rope_batch + tune_attn_causal_gqa_fwd):
//   rope_k    K -> RoPE -> k_rot (caller dtype) and/or a compute-dtype copy
//             (plus a bf16 copy of V when fp32 tensors feed bf16 matrix cores).
//   attn_fwd  fp32 mode: one workgroup = 64 queries of one head (this file);
//             bf16 mode: attn_fwd.hip (key-split waves, LDS DMA).  Q is
//             rotated on load (q_rot written if asked); online softmax in
//             fp32 (exp2 domain); O and the row log-sum-exp are written at
//             the end.  No [S,S] matrix exists.
// Backward (GpuLoraEngine.Backward.cs:354-412 dq_ds + dk_dv, :452 inverse rope):
//   attn_bwd  one launch with two kinds of workgroup.  dK/dV tiles: 64 keys of
//             one query head; dV_h = P^T dO and dK_h = scale dS^T Q accumulated
//             in registers over all query tiles, written as this head's fp32
//             partial.  dQ tiles: 64 queries of one head; P recomputed from
//             the saved lse, dS = P (dP - D), dQ = scale dS K, inverse RoPE on
//             the store.  Both form D_i = dO_i . O_i themselves.
//   attn_bwd_reduce  dK/dV = sum of the partials over the heads of the KV
//             group in ascending head order (the reference's workspace
//             reduction, CausalAttentionKernel.cs:184-206), inverse RoPE on dK.
// Every reduction has a fixed order and no kernel uses floating-point
// atomics, so results are bitwise repeatable (the activation-checkpoint
// recompute relies on that).
#include "attn_common.hpp"
#include "attn_launch.hpp"

#include <hip/hip_ext.h>

#include <type_traits>

namespace glacier {

// ---------------------------------------------------------------------------
// rope_k: grid (tokens * 8-pair chunks / 256, kv heads), one thread per
// (token, kv head, 8 rotation pairs); no division by a runtime value before
// the loads.  Writes the rotated K to k_rot (caller dtype) and/or kc
// (compute dtype), and, when vc is given, a compute-dtype copy of V.
// pos_of == nullptr: one sequence, the token index is the position (no table
// load before the cos/sin loads).
// ---------------------------------------------------------------------------
// The arguments its loads need come first (preloaded in SGPRs: build.py).
template <typename IO, typename T, int D>
__global__ __launch_bounds__(kThreads) void rope_k_kernel(
    const IO* __restrict__ k, const float* __restrict__ cos_t, const float* __restrict__ sin_t,
    const int32_t* __restrict__ pos_of, int total_tokens, int n_heads_kv, IO* __restrict__ k_rot,
    T* __restrict__ kc, const IO* __restrict__ v, T* __restrict__ vc) {
  constexpr int H = D / 2;
  constexpr int CH = H / 8;  // 8-pair chunks per head
  const int idx = blockIdx.x * kThreads + threadIdx.x;
  if (idx >= total_tokens * CH) return;
  const int tok = idx / CH, p0 = 8 * (idx % CH);
  const long base = ((long)tok * n_heads_kv + blockIdx.y) * D + p0;
  const long ti = (long)(pos_of != nullptr ? pos_of[tok] : tok) * H + p0;
  float x0[8], x1[8], c[8], s[8], y0[8], y1[8];
  load8(k + base, x0);
  load8(k + base + H, x1);
  load8(cos_t + ti, c);
  load8(sin_t + ti, s);
#pragma unroll
  for (int e = 0; e < 8; ++e) rope_fwd(x0[e], x1[e], c[e], s[e], y0[e], y1[e]);
  if (k_rot != nullptr) {
    store8(k_rot + base, y0);
    store8(k_rot + base + H, y1);
  }
  if (kc != nullptr) {
    store8(kc + base, y0);
    store8(kc + base + H, y1);
  }
  if (vc != nullptr) {
    load8(v + base, x0);
    load8(v + base + H, x1);
    store8(vc + base, x0);
    store8(vc + base + H, x1);
  }
}

// ---------------------------------------------------------------------------
// attn_fwd: grid (Hq, ntiles), 256 * G threads.  G key groups split a query
// tile's key tiles (group grp takes tiles grp, grp + G, ...): 2 in the bf16
// mode, so two waves share each SIMD and one's softmax arithmetic overlaps
// the other's matrix products; 1 in the fp32 mode (its tiles are twice as
// large).  Each group double-buffers its own K and V tiles in LDS; the
// groups' partial (max, sum, O) are merged through LDS at the end in a fixed
// order.  kc: rotated K in the compute dtype T; v: V in the caller's dtype.
// tiles == nullptr means one sequence of total_tokens tokens (the tile order
// is then computed, longest first, instead of read).
// ---------------------------------------------------------------------------
// Two key groups need a 64-row tile to split evenly over 512 threads' 8-element
// chunks (D a multiple of 64) and both groups' double buffers to fit the LDS
// (D <= 128); other head sizes take one group.
template <typename T, int D>
constexpr int fwd_groups() {
  return (sizeof(T) == 2 && D % 64 == 0 && D <= 128) ? 2 : 1;
}

// Lazy rescaling: the running max used for exp2 moves only when a tile's max
// exceeds it by more than this (log2 units), so P stays <= 2^8 and O is
// rescaled only a few times per row instead of once per tile.
constexpr float kRescaleTau = 8.0f;

template <typename IO, typename T, int D>
__global__ __launch_bounds__((kThreads * fwd_groups<T, D>())) void attn_fwd_kernel(
    const IO* __restrict__ q, const T* __restrict__ kc, const IO* __restrict__ v,
    IO* __restrict__ out, float* __restrict__ lse, IO* __restrict__ q_rot,
    const TileDesc* __restrict__ tiles, int n_tiles, int n_heads_q, int n_heads_kv,
    int total_tokens, float scale_log2, const float* __restrict__ cos_t,
    const float* __restrict__ sin_t) {
  using M = Mfma<T>;
  using L = Lds<T, D>;
  constexpr int G = fwd_groups<T, D>();
  constexpr int NKD = D / M::KSTEP;
  constexpr int H = D / 2;
  extern __shared__ __align__(16) unsigned char smem_raw[];
  T* const lds = reinterpret_cast<T*>(smem_raw);  // [G][2 buffers][K tile, V tile]

  const int h = blockIdx.x;
  const TileDesc td = tiles != nullptr
                          ? tiles[blockIdx.y]
                          : TileDesc{0, total_tokens, n_tiles - 1 - (int)blockIdx.y, 0};
  const int kvh = h / (n_heads_q / n_heads_kv);
  const int tid = threadIdx.x, w = wave_id(), lane = tid & 63;
  const int grp = w >> 2, wq = w & 3, gtid = tid & (kThreads - 1);
  const int g = lane >> 4, c = lane & 15;
  const int qrow = kTile * td.tile + 16 * wq + c;
  const bool qvalid = qrow < td.len;
  const long qbase = ((long)(td.tok0 + qrow) * n_heads_q + h) * D;
  T* const glds = lds + grp * 4 * L::TILE;  // this group's two buffers

  // Start this group's first K/V tile loads before the Q prologue.
  const long kvstride = (long)n_heads_kv * D;
  const T* kbase = kc + ((long)td.tok0 * n_heads_kv + kvh) * D;
  const IO* vbase = v + ((long)td.tok0 * n_heads_kv + kvh) * D;
  TileRegs<T, D> kreg;
  TileRegs<IO, D> vreg;
  if (grp <= td.tile) {
    const long roff = (long)kTile * grp * kvstride;
    kreg.load(kbase + roff, kvstride, td.len - kTile * grp, gtid);
    vreg.load(vbase + roff, kvstride, td.len - kTile * grp, gtid);
  }

  // Q fragments, rotated in fp32 then rounded to the compute dtype.  Group 0
  // rotates (and writes q_rot); with two groups it hands the fragments to
  // group 1 through LDS, lane for lane, so Q and the cos/sin rows are read
  // from memory once per workgroup.
  typename M::Frag qf[NKD];
  if constexpr (H % M::KSTEP != 0) {
    // Half the head is not a whole number of k-steps (bf16, D = 32 or 96):
    // each fragment's 8 elements (all on one side of H, as H % 8 == 0) are
    // rotated against their partner half on their own, with the same fp32
    // operations as the paired path.
    static_assert(sizeof(T) == 2 && H % 8 == 0 && G == 1, "per-fragment rotation layout");
#pragma unroll
    for (int kk = 0; kk < NKD; ++kk) {
      const int d0 = kk * M::KSTEP + 8 * g;
      const bool lo = d0 < H;
      const int dp = lo ? d0 + H : d0 - H;  // the partner half
      const int pi = lo ? d0 : d0 - H;      // the rotation pair
      float x[8], xp[8], cs[8], sn[8], y[8];
      if (qvalid) {
        load8(q + qbase + d0, x);
        load8(q + qbase + dp, xp);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) x[e] = xp[e] = 0.0f;
      }
      const long ti = (long)(qvalid ? qrow : 0) * H + pi;
      load8(cos_t + ti, cs);
      load8(sin_t + ti, sn);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        float y0, y1;
        if (lo) {
          rope_fwd(x[e], xp[e], cs[e], sn[e], y0, y1);
          y[e] = y0;
        } else {
          rope_fwd(xp[e], x[e], cs[e], sn[e], y0, y1);
          y[e] = y1;
        }
        qf[kk][e] = (bf16)y[e];
      }
      if (q_rot != nullptr && qvalid) store8(q_rot + qbase + d0, y);
    }
  } else if (grp == 0) {
#pragma unroll
    for (int kk = 0; kk < NKD / 2; ++kk) {
      if constexpr (sizeof(T) == 2) {
        const int d0 = kk * M::KSTEP + 8 * g;
        float x0[8], x1[8], y0[8], y1[8], cs[8], sn[8];
        if (qvalid) {
          load8(q + qbase + d0, x0);
          load8(q + qbase + d0 + H, x1);
        } else {
#pragma unroll
          for (int e = 0; e < 8; ++e) x0[e] = x1[e] = 0.0f;
        }
        const long ti = (long)(qvalid ? qrow : 0) * H + d0;
        load8(cos_t + ti, cs);
        load8(sin_t + ti, sn);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          rope_fwd(x0[e], x1[e], cs[e], sn[e], y0[e], y1[e]);
          qf[kk][e] = (bf16)y0[e];
          qf[kk + NKD / 2][e] = (bf16)y1[e];
        }
        if (q_rot != nullptr && qvalid) {
          store8(q_rot + qbase + d0, y0);
          store8(q_rot + qbase + d0 + H, y1);
        }
      } else {
        const int d0 = kk * M::KSTEP + g;
        float x0 = 0.0f, x1 = 0.0f, y0, y1;
        if (qvalid) {
          x0 = to_f32(q[qbase + d0]);
          x1 = to_f32(q[qbase + d0 + H]);
        }
        const long ti = (long)(qvalid ? qrow : 0) * H + d0;
        rope_fwd(x0, x1, cos_t[ti], sin_t[ti], y0, y1);
        qf[kk] = y0;
        qf[kk + NKD / 2] = y1;
        if (q_rot != nullptr && qvalid) {
          q_rot[qbase + d0] = from_f32<IO>(y0);
          q_rot[qbase + d0 + H] = from_f32<IO>(y1);
        }
      }
    }
  }
  typename M::Frag* const qlds =
      reinterpret_cast<typename M::Frag*>(lds + 4 * G * L::TILE) + wq * NKD * 64 + lane;
  if constexpr (G == 2) {
    if (grp == 0) {
#pragma unroll
      for (int kk = 0; kk < NKD; ++kk) qlds[kk * 64] = qf[kk];
    }
  }

  f32x4 o[D / 16];
#pragma unroll
  for (int db = 0; db < D / 16; ++db) o[db] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  float m_run = kNegBig, l_lane = 0.0f;

  // One key tile: scores, online softmax, O^T += V^T P^T.  DIAG: the tile
  // that holds the queries themselves (causal mask inside it).
  auto step = [&](const T* ks, const T* vs, auto diag) {
    constexpr bool DIAG = decltype(diag)::value;
    const int nb = DIAG ? (wq + 1) : 4;
    float sc[4][4];
    float mloc = -INFINITY;
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
      if (b < nb) {
#pragma unroll
        for (int kk = 0; kk < NKD; ++kk)
          acc = M::mma(frag_rm<T, D>(ks, 16 * b + c, kk, g), qf[kk], acc);
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        float x = acc[r];
        if (DIAG) x = (b < nb && 16 * b + 4 * g + r <= 16 * wq + c) ? x : -INFINITY;
        sc[b][r] = x;
        mloc = fmaxf(mloc, x);
      }
    }
    const float m_tile = col_max(mloc) * scale_log2;
    if (__builtin_amdgcn_ballot_w64(m_tile > m_run + kRescaleTau) != 0) {
      const float m_new = fmaxf(m_run, m_tile);
      const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
      l_lane *= alpha;
#pragma unroll
      for (int db = 0; db < D / 16; ++db) o[db] *= alpha;
      m_run = m_new;
    }
    float p[4][4];
    float psum = 0.0f;
#pragma unroll
    for (int b = 0; b < 4; ++b)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        p[b][r] = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[b][r], scale_log2, -m_run));
        psum += p[b][r];
      }
    l_lane += psum;
    acc_rows<T, D>(o, vs, p, nb, lane);
  };

  if (grp <= td.tile) {
    kreg.store(glds, gtid);
    vreg.store(glds + L::TILE, gtid);
  }
  __syncthreads();
  if constexpr (G == 2) {
    if (grp == 1) {
#pragma unroll
      for (int kk = 0; kk < NKD; ++kk) qf[kk] = qlds[kk * 64];
    }
  }

  const int nit = (td.tile + G) / G;  // iterations of group 0 (the most)
  for (int it = 0; it < nit; ++it) {
    const int kt = grp + G * it;
    const T* ks = glds + (it & 1) * 2 * L::TILE;
    const bool more = kt + G <= td.tile;
    if (more) {  // prefetch this group's next tile into registers
      const long roff = (long)kTile * (kt + G) * kvstride;
      const int nv = td.len - kTile * (kt + G);
      kreg.load(kbase + roff, kvstride, nv, gtid);
      vreg.load(vbase + roff, kvstride, nv, gtid);
    }
    if (kt < td.tile)
      step(ks, ks + L::TILE, std::false_type{});
    else if (kt == td.tile)
      step(ks, ks + L::TILE, std::true_type{});
    if (more) {
      T* nxt = glds + ((it + 1) & 1) * 2 * L::TILE;
      kreg.store(nxt, gtid);
      vreg.store(nxt + L::TILE, gtid);
    }
    __syncthreads();
  }

  if constexpr (G == 2) {
    // Merge group 1's partial row state into group 0 (lane for lane: waves
    // wq and wq + 4 own the same queries with the same lane layout).
    constexpr int NF = D / 4 + 2;  // floats per lane: O, max, sum
    float* cmb = reinterpret_cast<float*>(lds + 4 * L::TILE) + wq * NF * 64 + lane;
    if (grp == 1) {
      cmb[0] = m_run;
      cmb[64] = l_lane;
#pragma unroll
      for (int db = 0; db < D / 16; ++db)
#pragma unroll
        for (int r = 0; r < 4; ++r) cmb[(2 + 4 * db + r) * 64] = o[db][r];
    }
    __syncthreads();
    if (grp == 1) return;
    const float m1 = cmb[0], l1 = cmb[64];
    const float m_new = fmaxf(m_run, m1);
    const float a0 = __builtin_amdgcn_exp2f(m_run - m_new);
    const float a1 = __builtin_amdgcn_exp2f(m1 - m_new);
    l_lane = l_lane * a0 + l1 * a1;
#pragma unroll
    for (int db = 0; db < D / 16; ++db)
#pragma unroll
      for (int r = 0; r < 4; ++r) o[db][r] = o[db][r] * a0 + cmb[(2 + 4 * db + r) * 64] * a1;
    m_run = m_new;
  }

  const float l_tot = col_sum(l_lane);
  const float inv = 1.0f / l_tot;
  if (qvalid) {
#pragma unroll
    for (int db = 0; db < D / 16; ++db)
      store4(out + qbase + 16 * db + 4 * g, o[db] * inv);
    if (lse != nullptr && g == 0)
      lse[(long)h * total_tokens + td.tok0 + qrow] = (m_run + log2f(l_tot)) * kLn2;
  }
}

// ---------------------------------------------------------------------------
// Backward, two launches:
//   attn_bwd    grid (Hq/Hkv, Hkv, 2 ntiles).  z < ntiles: dK/dV of one
//               (query head, key tile), accumulated in registers over the
//               query tiles (fp32) and written as that head's partial in
//               the caller's tensor dtype (bf16 for bf16 tensors, halving the
//               partials' traffic both ways; fp32 for fp32 tensors, so the
//               group sum of the fp32-tensor path accumulates in fp32);
//               z >= ntiles: dQ of one (query head, query tile), inverse RoPE
//               applied on the store.  Both kinds form the row terms
//               D_i = dO_i . O_i of the query tiles they stage with the same
//               arithmetic (row_term), so neither waits for the other and one
//               launch runs them side by side: the CUs that finish short tiles
//               of one kind pick up tiles of the other.
//   attn_bwd_reduce  dK/dV = the group's partials summed in ascending head
//               order (CausalAttentionKernel.cs:184-206), inverse RoPE on dK.
// G groups of 4 waves split a tile's loop (2 in the bf16 mode, 1 in fp32);
// their partial sums are added in group order.
// ---------------------------------------------------------------------------
template <typename T, int D>
constexpr int bwd_groups() {
  return (sizeof(T) == 2 && D % 64 == 0 && D <= 128) ? 2 : 1;
}

// D_i = dO_i . O_i for register-staged dO/O tiles: the thread's chunk i (8
// elements of one row) is multiplied out in order, then the partial sums of
// the CPR lanes that hold the row are added in a fixed order.  Every lane of
// the row gets the same bits, and both backward tile kinds use this, so they
// agree bit for bit.
template <typename IO, int D, int NT>
__device__ inline float row_term(const TileRegs<IO, D, NT>& dreg, const TileRegs<IO, D, NT>& oreg,
                                 int i) {
  float xd[8], xo[8];
  load8(reinterpret_cast<const IO*>(&dreg.w[i][0]), xd);
  load8(reinterpret_cast<const IO*>(&oreg.w[i][0]), xo);
  float part = 0.0f;
#pragma unroll
  for (int e = 0; e < 8; ++e) part += xd[e] * xo[e];
  return lanes_sum<TileRegs<IO, D, NT>::LPR>(part);
}

// dQ of one (query head, query tile); z indexes the query tiles (longest
// first for a single sequence).
template <typename IO, typename T, int D>
__device__ inline void bwd_dq_tile(
    const TileDesc td, const IO* __restrict__ q_rot, const IO* __restrict__ d_out,
    const IO* __restrict__ out, const IO* __restrict__ k_rot, const IO* __restrict__ v,
    const float* __restrict__ lse, IO* __restrict__ dq, int total_tokens, float scale_log2,
    float scale, const float* __restrict__ cos_t, const float* __restrict__ sin_t) {
  using M = Mfma<T>;
  using L = Lds<T, D>;
  constexpr int G = bwd_groups<T, D>();
  constexpr int NKD = D / M::KSTEP;
  constexpr int H = D / 2;
  using Regs = TileRegs<IO, D, kThreads * G>;
  extern __shared__ __align__(16) unsigned char smem_raw[];
  T* const lds = reinterpret_cast<T*>(smem_raw);  // [G][2 buffers][K tile, V tile]
  float* const dsm = reinterpret_cast<float*>(lds + 4 * G * L::TILE);  // [64] row terms

  const int ratio = gridDim.x, n_heads_kv = gridDim.y, n_heads_q = ratio * n_heads_kv;
  const int kvh = blockIdx.y, h = kvh * ratio + blockIdx.x;
  const int tid = threadIdx.x, w = wave_id(), lane = tid & 63;
  GL_STAMP(kKernBwd, 0);
  GL_STAMP_VALUE(kKernBwd, 31, 100 + td.tile);
  const int grp = w >> 2, wq = w & 3, gtid = tid & (kThreads - 1);
  const int g = lane >> 4, c = lane & 15;
  const int qrow = kTile * td.tile + 16 * wq + c;
  const bool qvalid = qrow < td.len;
  T* const glds = lds + grp * 4 * L::TILE;

  const long kvstride = (long)n_heads_kv * D;
  const IO* kbase = k_rot + ((long)td.tok0 * n_heads_kv + kvh) * D;
  const IO* vbase = v + ((long)td.tok0 * n_heads_kv + kvh) * D;
  TileRegs<IO, D> kreg, vreg;
  if (grp <= td.tile) {
    const long roff = (long)kTile * grp * kvstride;
    kreg.load(kbase + roff, kvstride, td.len - kTile * grp, gtid);
    vreg.load(vbase + roff, kvstride, td.len - kTile * grp, gtid);
  }

  // This tile's Q, dO and O rows (all threads, coalesced): dO and O give
  // the row terms D_i; Q and dO go through LDS to become the waves' operand
  // fragments.
  const long qstride = (long)n_heads_q * D;
  const long trow = ((long)(td.tok0 + kTile * td.tile) * n_heads_q + h) * D;
  Regs qreg, dreg, oreg;
  qreg.load(q_rot + trow, qstride, td.len - kTile * td.tile, tid);
  dreg.load(d_out + trow, qstride, td.len - kTile * td.tile, tid);
  oreg.load(out + trow, qstride, td.len - kTile * td.tile, tid);
  // Q and dO staging: group 0's second buffer, first written at the end of
  // its first iteration.
  T* const stg = lds + 2 * L::TILE;
  GL_STAMP(kKernBwd, 1);
  typename M::Frag qf[NKD], df[NKD];
  const long si = (long)h * total_tokens + td.tok0 + qrow;
  const float lse_q = qvalid ? lse[si] : 0.0f;

  f32x4 acc_dq[D / 16];
#pragma unroll
  for (int db = 0; db < D / 16; ++db) acc_dq[db] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  float drow = 0.0f, nlse2 = 0.0f;  // set once the row terms are staged
  // One key tile: S, dP, P from lse, dS = P (dP - D), dQ^T += K^T dS^T.
  auto step = [&](const T* ks, const T* vs, auto diag, auto mid, auto after) {
    constexpr bool DIAG = decltype(diag)::value;
    const int nb = DIAG ? (wq + 1) : 4;
    float ds[4][4];
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      f32x4 sv = {0.0f, 0.0f, 0.0f, 0.0f}, dp = {0.0f, 0.0f, 0.0f, 0.0f};
      if (b < nb) {
#pragma unroll
        for (int kk = 0; kk < NKD; ++kk) {
          sv = M::mma(frag_rm<T, D>(ks, 16 * b + c, kk, g), qf[kk], sv);
          dp = M::mma(frag_rm<T, D>(vs, 16 * b + c, kk, g), df[kk], dp);
        }
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float pv = __builtin_amdgcn_exp2f(__builtin_fmaf(sv[r], scale_log2, nlse2));
        float x = pv * (dp[r] - drow);
        if (DIAG) x = (b < nb && 16 * b + 4 * g + r <= 16 * wq + c) ? x : 0.0f;
        ds[b][r] = x;
      }
    }
    mid();
    acc_rows<T, D>(acc_dq, ks, ds, nb, lane);
    after();
  };

  if (grp <= td.tile) {
    kreg.store(glds, gtid);
    vreg.store(glds + L::TILE, gtid);
  }
  qreg.store(stg, tid);
  dreg.store(stg + L::TILE, tid);
#pragma unroll
  for (int i = 0; i < Regs::N; ++i) {
    const float part = row_term(dreg, oreg, i);
    const int idx = tid + i * kThreads * G;
    if (idx % Regs::LPR == 0) dsm[idx / Regs::LPR] = part;
  }
  wait_vmem_all();
  __syncthreads();
#pragma unroll
  for (int kk = 0; kk < NKD; ++kk) {
    qf[kk] = frag_rm<T, D>(stg, 16 * wq + c, kk, g);
    df[kk] = frag_rm<T, D>(stg + L::TILE, 16 * wq + c, kk, g);
  }
  drow = qvalid ? dsm[16 * wq + c] : 0.0f;
  nlse2 = qvalid ? -lse_q * kLog2e : 0.0f;
  __syncthreads();  // the staging area is free again
  GL_STAMP(kKernBwd, 2);

  const int nit = (td.tile + G) / G;
  auto iteration = [&](int it, auto diag, auto mid) {
    const int kt = grp + G * it;
    const T* ks = glds + (it & 1) * 2 * L::TILE;
    const bool more = kt + G <= td.tile;
    auto prefetch = [&] {
      if (more) {
        const long roff = (long)kTile * (kt + G) * kvstride;
        const int nv = td.len - kTile * (kt + G);
        kreg.load(kbase + roff, kvstride, nv, gtid);
        vreg.load(vbase + roff, kvstride, nv, gtid);
      }
    };
    // The next tile's loads: for bf16 tensors at the end of this tile's step
    // (issued first, they stall the wave while the memory pipeline is full;
    // more implies kt < td.tile, so the step runs whenever they are due),
    // for fp32 tensors up front (the registers fp32 tile loads hold across
    // the step would not fit beside its products).
    if constexpr (sizeof(IO) == 4) prefetch();
    if (decltype(diag)::value || kt < td.tile)
      step(ks, ks + L::TILE, diag, mid, [&] {
        if constexpr (sizeof(IO) != 4) prefetch();
      });
    else
      mid();  // a group with no tile left in this iteration
    if (it < 6) GL_STAMP(kKernBwd, 3 + 3 * it);
    if (more) {
      T* nxt = glds + ((it + 1) & 1) * 2 * L::TILE;
      kreg.store(nxt, gtid);
      vreg.store(nxt + L::TILE, gtid);
    }
    if (it < 6) GL_STAMP(kKernBwd, 4 + 3 * it);
    __syncthreads();
    if (it < 6) GL_STAMP(kKernBwd, 5 + 3 * it);
  };
  // Every iteration but the last takes a key tile below the diagonal; the
  // diagonal tile is the last iteration of one group.  Peeling it keeps a
  // single step variant inside the loop (two variants in one loop body make
  // the register allocator copy the loop-carried registers every iteration).
  for (int it = 0; it + 1 < nit; ++it) iteration(it, std::false_type{}, [] {});
  // The epilogue scales dQ, applies the inverse RoPE at the query's
  // position and stores whole rows.  Rotation block p holds the lane's
  // d = 16 p + 4 g + 0..3 (acc_dq[p]) and d + D/2 (acc_dq[p + NP]); with
  // two groups, each finishes half of the blocks (group 0 the first half)
  // after adding the other group's accumulators for them, received through
  // LDS (group 0's sum first either way).  The blocks' cos/sin values: for
  // bf16 tensors loaded inside the last iteration's step (between its dS
  // block and its product; that iteration has no next tile to load), so the
  // step hides their latency; fp32 tensors load them in the epilogue (held
  // across the step, they would not fit beside the fp32 tile registers).
  constexpr int NP = D / 32;  // rotation blocks
  constexpr int PB = NP / G;  // blocks each group finishes
  constexpr bool kEarlyRope = sizeof(IO) != 4;
  f32x4 rc[PB], rs[PB];
  const long ti0 = (long)(qvalid ? qrow : 0) * H + 16 * PB * grp + 4 * g;
  auto load_rope = [&] {
#pragma unroll
    for (int j = 0; j < PB; ++j) {
      rc[j] = *reinterpret_cast<const f32x4*>(cos_t + ti0 + 16 * j);
      rs[j] = *reinterpret_cast<const f32x4*>(sin_t + ti0 + 16 * j);
    }
  };
  auto rope_mid = [&] {
    if (kEarlyRope) load_rope();
  };
  if (grp + G * (nit - 1) == td.tile)
    iteration(nit - 1, std::true_type{}, rope_mid);
  else
    iteration(nit - 1, std::false_type{}, rope_mid);

  GL_STAMP(kKernBwd, 21);
  // GR: the group as a constant (accumulators are indexed at compile time)
  f32x4* const cx = reinterpret_cast<f32x4*>(lds + 4 * L::TILE);  // [G][4 waves][2 PB][64 lanes]
  auto hand_over = [&](auto grc) {
    constexpr int GR = decltype(grc)::value;
    f32x4* const o = cx + (GR * 4 + wq) * 2 * PB * 64 + lane;
#pragma unroll
    for (int j = 0; j < PB; ++j) {
      o[2 * j * 64] = acc_dq[(1 - GR) * PB + j];
      o[(2 * j + 1) * 64] = acc_dq[(1 - GR) * PB + j + NP];
    }
  };
  // The [64][D] dQ tile is staged in LDS in the output dtype (row stride
  // D + 8), then every thread stores 16-byte pieces of consecutive rows,
  // streamed (store16_nt), like the dK/dV partials: at S=512 that shortened
  // the step by 0.5-0.7 µs at most head counts (the kernel no longer ends on
  // the write-back of its dirty L2 lines).
  constexpr int SR = D + 8;
  IO* const stq = reinterpret_cast<IO*>(smem_raw);
  auto finish = [&](auto grc) {
    constexpr int GR = decltype(grc)::value;
    if constexpr (G == 2) {
      const f32x4* const in = cx + ((1 - GR) * 4 + wq) * 2 * PB * 64 + lane;
#pragma unroll
      for (int j = 0; j < PB; ++j) {
        acc_dq[GR * PB + j] += in[2 * j * 64];
        acc_dq[GR * PB + j + NP] += in[(2 * j + 1) * 64];
      }
    }
    if (!kEarlyRope) load_rope();
#pragma unroll
    for (int j = 0; j < PB; ++j) {
      const int pb = GR * PB + j;
      const f32x4 lo = acc_dq[pb] * scale, hi = acc_dq[pb + NP] * scale;
      const int d0 = 16 * pb + 4 * g;
      f32x4 y0, y1;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        float a, b;
        rope_inv(lo[r], hi[r], rc[j][r], rs[j][r], a, b);
        y0[r] = a;
        y1[r] = b;
      }
      store4(stq + (16 * wq + c) * SR + d0, y0);
      store4(stq + (16 * wq + c) * SR + H + d0, y1);
    }
  };
  if constexpr (G == 2) {
    if (grp == 0)
      hand_over(std::integral_constant<int, 0>{});
    else
      hand_over(std::integral_constant<int, 1>{});
    __syncthreads();
    GL_STAMP(kKernBwd, 23);
    if (grp == 0)
      finish(std::integral_constant<int, 0>{});
    else
      finish(std::integral_constant<int, 1>{});
  } else {
    finish(std::integral_constant<int, 0>{});
  }
  __syncthreads();
  GL_STAMP(kKernBwd, 24);
  constexpr int EPC = 16 / sizeof(IO);  // elements per 16-byte piece
  constexpr int PPR = D / EPC;          // pieces per row
#pragma unroll
  for (int i = tid; i < kTile * PPR; i += kThreads * G) {
    const int r = i / PPR, pc = i % PPR;
    if (kTile * td.tile + r < td.len)
      store16_nt(dq + ((long)(td.tok0 + kTile * td.tile + r) * n_heads_q + h) * D + pc * EPC,
                 stq + r * SR + pc * EPC);
  }
  GL_STAMP(kKernBwd, 22);
}

// dK/dV partial of one (query head, key tile); z indexes the key tiles.
template <typename IO, typename T, int D>
__device__ inline void bwd_dkdv_tile(
    const TileDesc td, const IO* __restrict__ q_rot, const IO* __restrict__ d_out,
    const IO* __restrict__ out, const IO* __restrict__ k_rot, const IO* __restrict__ v,
    const float* __restrict__ lse, IO* __restrict__ wk, IO* __restrict__ wv,
    int total_tokens, float scale_log2, float scale) {
  using M = Mfma<T>;
  using L = Lds<T, D>;
  using Regs = TileRegs<IO, D>;
  constexpr int G = bwd_groups<T, D>();
  constexpr int NKD = D / M::KSTEP;
  constexpr int BUF = 2 * L::TILE * sizeof(T) + 2 * kTile * sizeof(float);  // bytes
  extern __shared__ __align__(16) unsigned char smem_raw[];

  const int ratio = gridDim.x, n_heads_kv = gridDim.y, n_heads_q = ratio * n_heads_kv;
  const int kvh = blockIdx.y, h = kvh * ratio + blockIdx.x;
  const int tid = threadIdx.x, w = wave_id(), lane = tid & 63;
  GL_STAMP(kKernBwd, 0);
  GL_STAMP_VALUE(kKernBwd, 31, td.tile);
  const int grp = w >> 2, wq = w & 3, gtid = tid & (kThreads - 1);
  const int g = lane >> 4, c = lane & 15;
  unsigned char* const gsm = smem_raw + grp * 2 * BUF;

  const int ntq = (td.len + kTile - 1) / kTile;
  // the query tiles this entry visits: all from the diagonal one, or one half
  const QueryRange qr = dkdv_query_range(td.tile, ntq, td.kind);
  const long qstride = (long)n_heads_q * D;
  const IO* qb = q_rot + ((long)td.tok0 * n_heads_q + h) * D;
  const IO* dob = d_out + ((long)td.tok0 * n_heads_q + h) * D;
  const IO* ob = out + ((long)td.tok0 * n_heads_q + h) * D;
  const float* lseb = lse + (long)h * total_tokens + td.tok0;

  // Stage one query tile: Q, dO and O rows into registers, -lse*log2(e)
  // (-inf past the sequence, so P and dS are 0 there) into one float.
  // The loaded lse is used only when the tile is stored: any arithmetic on
  // it here would make the wave wait for every load just issued (loads
  // complete in order), exposing the prefetch instead of hiding it.
  Regs qreg, dreg, oreg;
  float lse_raw = 0.0f;
  auto load_tile = [&](int qt) {
    const long roff = (long)kTile * qt * qstride;
    const int nv = td.len - kTile * qt;
    qreg.load(qb + roff, qstride, nv, gtid);
    dreg.load(dob + roff, qstride, nv, gtid);
    oreg.load(ob + roff, qstride, nv, gtid);
    if (gtid < kTile && gtid < nv) lse_raw = lseb[kTile * qt + gtid];
  };
  // ... and write it to LDS buffer `buf` with the row terms D_i.
  auto store_tile = [&](int buf, int qt) {
    unsigned char* base = gsm + buf * BUF;
    qreg.store(reinterpret_cast<T*>(base), gtid);
    dreg.store(reinterpret_cast<T*>(base) + L::TILE, gtid);
    float* vec = reinterpret_cast<float*>(base + 2 * L::TILE * sizeof(T));
    if (gtid < kTile) vec[gtid] = gtid < td.len - kTile * qt ? -lse_raw * kLog2e : -INFINITY;
#pragma unroll
    for (int i = 0; i < Regs::N; ++i) {
      const float part = row_term(dreg, oreg, i);
      const int idx = gtid + i * kThreads;
      if (idx % Regs::LPR == 0) vec[kTile + idx / Regs::LPR] = part;
    }
  };

  // The key tile's K and V rows (all threads, coalesced), staged in group
  // 0's second buffer (first written at the end of its first iteration) and
  // read back as the waves' operand fragments; then each group's first query
  // tile.
  using KRegs = TileRegs<IO, D, kThreads * G>;
  KRegs kst, vst;
  {
    const long krow0 = ((long)(td.tok0 + kTile * td.tile) * n_heads_kv + kvh) * D;
    const long kvstride = (long)n_heads_kv * D;
    kst.load(k_rot + krow0, kvstride, td.len - kTile * td.tile, tid);
    vst.load(v + krow0, kvstride, td.len - kTile * td.tile, tid);
  }
  const int first = qr.first + grp;
  if (first < qr.end) load_tile(first);
  GL_STAMP(kKernBwd, 1);
  T* const kvs = reinterpret_cast<T*>(smem_raw + BUF);
  kst.store(kvs, tid);
  vst.store(kvs + L::TILE, tid);
  typename M::Frag kf[NKD], vf[NKD];

  f32x4 acc_dk[D / 16], acc_dv[D / 16];
#pragma unroll
  for (int db = 0; db < D / 16; ++db) {
    acc_dk[db] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    acc_dv[db] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  }

  // One query tile: S, dP (keys as columns), P, dS; dV^T += dO^T P,
  // dK^T += Q^T dS.  DIAG: the query tile that holds the keys themselves.
  auto step = [&](const unsigned char* base, auto diag, auto mid) {
    constexpr bool DIAG = decltype(diag)::value;
    const T* qs = reinterpret_cast<const T*>(base);
    const T* dos = qs + L::TILE;
    const float* nlse_s = reinterpret_cast<const float*>(base + 2 * L::TILE * sizeof(T));
    const float* d_s = nlse_s + kTile;
    const int b0 = DIAG ? wq : 0;  // query blocks below b0 are masked
    float p[4][4], ds[4][4];
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      f32x4 sv = {0.0f, 0.0f, 0.0f, 0.0f}, dp = {0.0f, 0.0f, 0.0f, 0.0f};
      if (b >= b0) {
#pragma unroll
        for (int kk = 0; kk < NKD; ++kk) {
          sv = M::mma(frag_rm<T, D>(qs, 16 * b + c, kk, g), kf[kk], sv);
          dp = M::mma(frag_rm<T, D>(dos, 16 * b + c, kk, g), vf[kk], dp);
        }
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int qi = 16 * b + 4 * g + r;
        float pv = __builtin_amdgcn_exp2f(__builtin_fmaf(sv[r], scale_log2, nlse_s[qi]));
        if (DIAG) pv = (b >= b0 && 16 * wq + c <= qi) ? pv : 0.0f;
        p[b][r] = pv;
        ds[b][r] = pv * (dp[r] - d_s[qi]);
      }
    }
    acc_rows<T, D>(acc_dv, dos, p, 4, lane);
    mid();
    acc_rows<T, D>(acc_dk, qs, ds, 4, lane);
  };

  if (first < qr.end) store_tile(0, first);
  wait_vmem_all();
  __syncthreads();
#pragma unroll
  for (int kk = 0; kk < NKD; ++kk) {
    kf[kk] = frag_rm<T, D>(kvs, 16 * wq + c, kk, g);
    vf[kk] = frag_rm<T, D>(kvs + L::TILE, 16 * wq + c, kk, g);
  }
  __syncthreads();  // the staging area is free again
  GL_STAMP(kKernBwd, 2);

  const int nit = (qr.end - qr.first + G - 1) / G;  // iterations of group 0 (the most)
  auto iteration = [&](int it, auto diag) {
    const int qt = first + G * it;
    const unsigned char* base = gsm + (it & 1) * BUF;
    const bool more = qt + G < qr.end;
    // The next tile's loads: for bf16 tensors between this tile's dV and dK
    // products (issued first, they stall the wave while the memory pipeline
    // is full; more implies qt < qr.end, so the step runs whenever they are
    // due), for fp32 tensors up front (the registers fp32 tile loads hold
    // across the step would not fit beside its products).
    if (sizeof(IO) == 4 && more) load_tile(qt + G);
    if (qt < qr.end) step(base, diag, [&] {
      if (sizeof(IO) != 4 && more) load_tile(qt + G);
    });
    if (it < 6) GL_STAMP(kKernBwd, 3 + 3 * it);
    if (more) store_tile((it + 1) & 1, qt + G);
    if (it < 6) GL_STAMP(kKernBwd, 4 + 3 * it);
    __syncthreads();
    if (it < 6) GL_STAMP(kKernBwd, 5 + 3 * it);
  };
  // The diagonal query tile (when this entry visits it) is group 0's first
  // iteration; peeling it keeps a single step variant inside the loop (two
  // variants in one loop body make the register allocator copy the
  // accumulators every iteration).
  int it0 = 0;
  if (grp == 0 && nit > 0 && qr.first == td.tile) {
    iteration(0, std::true_type{});
    it0 = 1;
  }
  for (int it = it0; it < nit; ++it) iteration(it, std::false_type{});

  GL_STAMP(kKernBwd, 21);
  // Merge the groups and write whole rows.  Group 0 hands its fp32 dK
  // accumulators to group 1 through LDS and group 1 its dV to group 0 (row
  // stride D + 4 floats, so the 16 key rows of a wave's store fall in
  // distinct banks); each group adds the other's half to its own (group 0's
  // sum first either way) and stages that tensor's [64 keys][D] rows in the
  // partials' dtype, so the row stores read a quarter of the fp32 bytes
  // back for bf16.  Then every thread stores 16-byte pieces of consecutive
  // rows (streamed, as dQ).  Lane (g, c) holds d = 16 db + 4 g + 0..3 of
  // key 16 wq + c.
  constexpr int SR = D + 4;
  constexpr int SRO = D + (sizeof(IO) == 4 ? 4 : 8);  // row stride of the staged rows
  constexpr size_t MERGE = G == 2 ? 2 * kTile * SR * sizeof(float) : 0;
  static_assert(MERGE + 2 * kTile * SRO * sizeof(IO) <= 2 * BUF * G, "staging exceeds the LDS buffers");
  float* const stk = reinterpret_cast<float*>(smem_raw);
  float* const stv = stk + kTile * SR;
  IO* const sok = reinterpret_cast<IO*>(smem_raw + MERGE);
  IO* const sov = sok + kTile * SRO;
  IO* const ok = sok + (16 * wq + c) * SRO + 4 * g;
  IO* const ov = sov + (16 * wq + c) * SRO + 4 * g;
  if constexpr (G == 2) {
    f32x4* const pk = reinterpret_cast<f32x4*>(stk + (16 * wq + c) * SR + 4 * g);
    f32x4* const pv = reinterpret_cast<f32x4*>(stv + (16 * wq + c) * SR + 4 * g);
    if (grp == 0) {
#pragma unroll
      for (int db = 0; db < D / 16; ++db) pk[4 * db] = acc_dk[db];
    } else {
#pragma unroll
      for (int db = 0; db < D / 16; ++db) pv[4 * db] = acc_dv[db];
    }
    __syncthreads();
    GL_STAMP(kKernBwd, 23);
    if (grp == 0) {
#pragma unroll
      for (int db = 0; db < D / 16; ++db) store4(ov + 16 * db, acc_dv[db] + pv[4 * db]);
    } else {
#pragma unroll
      for (int db = 0; db < D / 16; ++db) store4(ok + 16 * db, (pk[4 * db] + acc_dk[db]) * scale);
    }
  } else {
#pragma unroll
    for (int db = 0; db < D / 16; ++db) {
      store4(ok + 16 * db, acc_dk[db] * scale);
      store4(ov + 16 * db, acc_dv[db]);
    }
  }
  __syncthreads();
  GL_STAMP(kKernBwd, 24);
  constexpr int EPC = 16 / sizeof(IO);  // elements per 16-byte piece
  constexpr int PPR = D / EPC;          // pieces per row
#pragma unroll
  for (int i = tid; i < kTile * PPR; i += kThreads * G) {
    const int r = i / PPR, pc = i % PPR;
    const int key = kTile * td.tile + r;
    if (key < td.len) {
      const long wb = ((long)(td.tok0 + key) * n_heads_q + h) * D + pc * EPC;
      store16_nt(wk + wb, sok + r * SRO + pc * EPC);
      store16_nt(wv + wb, sov + r * SRO + pc * EPC);
    }
  }
  GL_STAMP(kKernBwd, 22);
}

// z indexes tiles_bwd, the dK/dV (whole or half) and dQ tiles in launch order.  The
// table is read through the scalar cache (one uniform load per workgroup).
template <typename IO, typename T, int D>
__global__ __launch_bounds__((kThreads * bwd_groups<T, D>())) void attn_bwd_kernel(
    const TileDesc* __restrict__ tiles_bwd, const IO* __restrict__ q_rot,
    const IO* __restrict__ d_out, const IO* __restrict__ out, const IO* __restrict__ k_rot,
    const IO* __restrict__ v, int total_tokens, float scale_log2, const float* __restrict__ lse,
    IO* __restrict__ dq, IO* __restrict__ wk, IO* __restrict__ wv, IO* __restrict__ wk2,
    IO* __restrict__ wv2, float scale, const float* __restrict__ cos_t,
    const float* __restrict__ sin_t) {
  const TileDesc td = tiles_bwd[blockIdx.z];
  if (td.kind == kTileDq) {
    bwd_dq_tile<IO, T, D>(td, q_rot, d_out, out, k_rot, v, lse, dq, total_tokens, scale_log2,
                          scale, cos_t, sin_t);
  } else {
    // the second half of a split tile writes the second partials
    const bool second = td.kind == kTileDkDvSecondHalf;
    bwd_dkdv_tile<IO, T, D>(td, q_rot, d_out, out, k_rot, v, lse, second ? wk2 : wk,
                            second ? wv2 : wv, total_tokens, scale_log2, scale);
  }
#ifdef GLACIER_PHASE_STAMPS
  // profiling builds: the workgroup's end (its last wave's) and where it ran
  // (HW_ID: CU, shader array, engine; XCC_ID)
  __syncthreads();
  GL_STAMP(kKernBwd, 25);
  GL_STAMP_VALUE(kKernBwd, 26, __builtin_amdgcn_s_getreg((31 << 11) | 4));
  GL_STAMP_VALUE(kKernBwd, 27, __builtin_amdgcn_s_getreg((31 << 11) | 20));
#endif
}

// Threads of a reduction workgroup; each finishes 4 rotation pairs of one
// (token, kv head) row, so a workgroup covers kRedThreads / (D / 8) rows.
constexpr int kRedThreads = 128;

// 4 consecutive partial elements (the tensors' dtype) as fp32.
__device__ inline f32x4 load_partial4(const float* p) { return *reinterpret_cast<const f32x4*>(p); }
__device__ inline f32x4 load_partial4(const bf16* p) {
  const bf16x4 v = *reinterpret_cast<const bf16x4*>(p);
  return f32x4{(float)v[0], (float)v[1], (float)v[2], (float)v[3]};
}

// SPLIT: the call split dK/dV tiles (bf16 partials), so rows below
// split_rows have second partials.  hstep: the partials sit at every
// hstep-th head of the group (2 after the wide backward's head pairs).
// The arguments its loads need come first (preloaded in SGPRs: build.py).
template <typename IO, typename T, int D, bool SPLIT>
__global__ __launch_bounds__(kRedThreads) void attn_bwd_reduce_kernel(
    const IO* __restrict__ wk, const IO* __restrict__ wv, const int32_t* __restrict__ pos_of,
    const float* __restrict__ cos_t, const float* __restrict__ sin_t, int total_tokens, int ratio,
    int n_heads_kv, int hstep, IO* __restrict__ dk, IO* __restrict__ dv,
    const IO* __restrict__ wk2, const IO* __restrict__ wv2, int split_rows) {
  constexpr int H = D / 2;
  constexpr int CH = H / 4;  // 4-pair chunks per row
  constexpr int ROWS = kRedThreads / CH;
  GL_STAMP(kKernReduce, 0);
  if ((int)threadIdx.x >= ROWS * CH) return;  // CH need not divide the workgroup
  // grid (tokens / ROWS, kv heads): no division by a runtime value
  const int tok = blockIdx.x * ROWS + threadIdx.x / CH;
  if (tok >= total_tokens) return;
  const int p0 = 4 * (threadIdx.x % CH);
  const int j = blockIdx.y;  // kv head
  const long row = (long)tok * n_heads_kv + j;
  const int n_heads_q = ratio * n_heads_kv;
  const long pos = pos_of != nullptr ? pos_of[tok] : tok;
  const f32x4 cs = *reinterpret_cast<const f32x4*>(cos_t + pos * H + p0);
  const f32x4 sn = *reinterpret_cast<const f32x4*>(sin_t + pos * H + p0);
  const IO* wkr = wk + ((long)tok * n_heads_q + (long)j * ratio) * D + p0;
  const IO* wvr = wv + ((long)tok * n_heads_q + (long)j * ratio) * D + p0;
  // A row of a split dK/dV tile (bf16 partials only) has a second partial
  // per head, added right after the head's first.
  const bool two = SPLIT && pos < split_rows;
  const IO* wkr2 = wk2 + ((long)tok * n_heads_q + (long)j * ratio) * D + p0;
  const IO* wvr2 = wv2 + ((long)tok * n_heads_q + (long)j * ratio) * D + p0;
  f32x4 k0 = {0.0f, 0.0f, 0.0f, 0.0f}, k1 = k0, v0 = k0, v1 = k0;
  constexpr int RMAX = 8;
  constexpr int RMAX2 = SPLIT ? RMAX : 1;
  const int nparts = (ratio + hstep - 1) / hstep;  // partials per row, at heads 0, hstep, ..
  if (nparts <= RMAX) {
    // Every head's partial in flight at once (a load per head that the sum
    // waits on would cost one memory round trip per head), then the sum in
    // ascending head order; heads past the group add nothing.
    f32x4 pk0[RMAX], pk1[RMAX], pv0[RMAX], pv1[RMAX];
    f32x4 qk0[RMAX2], qk1[RMAX2], qv0[RMAX2], qv1[RMAX2];
#pragma unroll
    for (int hh = 0; hh < RMAX; ++hh) {
      const long o = (long)(hh < nparts ? hh * hstep : 0) * D;
      pk0[hh] = load_partial4(wkr + o);
      pk1[hh] = load_partial4(wkr + o + H);
      pv0[hh] = load_partial4(wvr + o);
      pv1[hh] = load_partial4(wvr + o + H);
    }
    if constexpr (RMAX2 == RMAX) {
      if (two) {
#pragma unroll
        for (int hh = 0; hh < RMAX; ++hh) {
          const long o = (long)(hh < ratio ? hh : 0) * D;
          qk0[hh] = load_partial4(wkr2 + o);
          qk1[hh] = load_partial4(wkr2 + o + H);
          qv0[hh] = load_partial4(wvr2 + o);
          qv1[hh] = load_partial4(wvr2 + o + H);
        }
      }
    }
#pragma unroll
    for (int hh = 0; hh < RMAX; ++hh) {
      if (hh < nparts) {
        k0 += pk0[hh];
        k1 += pk1[hh];
        v0 += pv0[hh];
        v1 += pv1[hh];
        if constexpr (RMAX2 == RMAX) {
          if (two) {
            k0 += qk0[hh];
            k1 += qk1[hh];
            v0 += qv0[hh];
            v1 += qv1[hh];
          }
        }
      }
    }
  } else {
    for (int hh = 0; hh < ratio; hh += hstep) {
      k0 += load_partial4(wkr + (long)hh * D);
      k1 += load_partial4(wkr + (long)hh * D + H);
      v0 += load_partial4(wvr + (long)hh * D);
      v1 += load_partial4(wvr + (long)hh * D + H);
      if (two) {
        k0 += load_partial4(wkr2 + (long)hh * D);
        k1 += load_partial4(wkr2 + (long)hh * D + H);
        v0 += load_partial4(wvr2 + (long)hh * D);
        v1 += load_partial4(wvr2 + (long)hh * D + H);
      }
    }
  }
  f32x4 y0, y1;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    float a, b;
    rope_inv(k0[e], k1[e], cs[e], sn[e], a, b);
    y0[e] = a;
    y1[e] = b;
  }
  const long dst = row * D + p0;
  store4(dk + dst, y0);
  store4(dk + dst + H, y1);
  store4(dv + dst, v0);
  store4(dv + dst + H, v1);
  GL_STAMP(kKernReduce, 22);
}

// ---------------------------------------------------------------------------
// Host launchers
// ---------------------------------------------------------------------------
namespace {

template <typename T, int D>
constexpr size_t fwd_lds() {
  // K/V double buffers per group, plus group 0's Q fragments for group 1
  return sizeof(T) * 4 * Lds<T, D>::TILE * fwd_groups<T, D>() +
         (fwd_groups<T, D>() == 2 ? sizeof(T) * kTile * D : 0);
}
template <typename T, int D>
constexpr size_t bwd_lds() {
  // dQ tiles: K/V double buffers per group plus the 64 row terms; dK/dV
  // tiles: Q/dO double buffers per group with the lse and D vectors.
  constexpr size_t dq = sizeof(T) * 4 * Lds<T, D>::TILE * bwd_groups<T, D>() + kTile * sizeof(float);
  constexpr size_t dkdv =
      2 * (sizeof(T) * 2 * Lds<T, D>::TILE + 2 * kTile * sizeof(float)) * bwd_groups<T, D>();
  return dq > dkdv ? dq : dkdv;
}

template <typename IO, typename T, int D>
hipError_t forward_impl(const FwdLaunch& a, hipStream_t st, KernelTimer* tm) {
  const dim3 blk(kThreads);
  T* kc = static_cast<T*>(a.kc);
  {
    const long n = (long)a.total_tokens * (D / 16);
    const dim3 grid(static_cast<unsigned>((n + kThreads - 1) / kThreads), a.n_heads_kv);
    IO* k_rot = static_cast<IO*>(a.k_rot);
    LaunchTiming t(tm, kKernRopeK);
    GL_LAUNCH(t, (rope_k_kernel<IO, T, D>), grid, blk, 0, st,
                          static_cast<const IO*>(a.k), a.cos_t, a.sin_t,
                          a.single_seq ? nullptr : a.pos_of, a.total_tokens, a.n_heads_kv, k_rot,
                          (static_cast<void*>(kc) == static_cast<void*>(k_rot)) ? nullptr : kc,
                          static_cast<const IO*>(a.v), static_cast<T*>(a.vc));
    GL_CHECK(hipGetLastError());
    t.launched();
  }
  if constexpr (sizeof(T) == 2 && (D == 64 || D == 128)) {
    GL_CHECK((launch_fwd_bf16<IO, D>(a, st, tm)));
  } else {
    auto fn = attn_fwd_kernel<IO, T, D>;
    constexpr size_t lds = fwd_lds<T, D>();
    GL_CHECK(allow_lds(fn, lds));
    LaunchTiming t(tm, kKernFwd);
    GL_LAUNCH(t, fn, dim3(a.n_heads_q, a.n_tiles), dim3(kThreads * fwd_groups<T, D>()), lds,
                          st, static_cast<const IO*>(a.q),
                          static_cast<const T*>(kc), static_cast<const IO*>(a.v),
                          static_cast<IO*>(a.out), a.lse, static_cast<IO*>(a.q_rot),
                          a.single_seq ? nullptr : a.tiles_fwd, a.n_tiles, a.n_heads_q,
                          a.n_heads_kv, a.total_tokens, a.scale_log2, a.cos_t, a.sin_t);
    GL_CHECK(hipGetLastError());
    t.launched();
  }
  return hipSuccess;
}

template <typename IO, typename T, int D>
hipError_t backward_impl(const BwdLaunch& a, hipStream_t st, KernelTimer* tm) {
  const int ratio = a.n_heads_q / a.n_heads_kv;
  bool rows32 = false, mfma32 = false;
  if constexpr (std::is_same<IO, bf16>::value && (D == 64 || D == 128)) {
    const long long min_work = D == 128 ? kBwdMfma32MinWorkD128 : kBwdMfma32MinWorkD64;
    mfma32 = a.tiles_wide != nullptr &&
             (a.variant == kBwdMfma32 ||
              (a.variant == kBwdAuto && a.pairs * a.n_heads_q >= min_work));
    rows32 = !mfma32 && a.variant == kBwdRows32;
  }
  if (mfma32) {
    // bf16 tensors: the 32x32x16-MFMA kernel (attn_bwd3.hip)
    if constexpr (D == 64 || D == 128) GL_CHECK(launch_bwd3<D>(a, st, tm));
    rows32 = true;  // no split tiles, whole-tile reduction
  } else if (rows32) {
    // bf16 tensors, long sequences: the 32-row-wave kernel fed by LDS DMA
    // (attn_bwd.hip; head_dim 64 and 128)
    if constexpr (D == 64 || D == 128) GL_CHECK(launch_bwd2<D>(a, st, tm));
  }
  // dK/dV tiles split in query halves: 16-row kernel, bf16 partials
  const bool split = !rows32 && sizeof(IO) == 2 && a.split > 0;
  if (!rows32) {
    auto fn = attn_bwd_kernel<IO, T, D>;
    constexpr size_t lds = bwd_lds<T, D>();
    GL_CHECK(allow_lds(fn, lds));
    LaunchTiming t(tm, kKernBwd);
    GL_LAUNCH(t, fn, dim3(ratio, a.n_heads_kv, split ? a.n_split_entries : 2 * a.n_tiles),
                          dim3(kThreads * bwd_groups<T, D>()), lds, st,
                          split ? a.tiles_split : a.tiles_bwd, static_cast<const IO*>(a.q_rot),
                          static_cast<const IO*>(a.d_out), static_cast<const IO*>(a.out),
                          static_cast<const IO*>(a.k_rot), static_cast<const IO*>(a.v),
                          a.total_tokens, a.scale_log2, a.lse, static_cast<IO*>(a.dq),
                          static_cast<IO*>(a.wk), static_cast<IO*>(a.wv),
                          static_cast<IO*>(split ? a.wk2 : nullptr),
                          static_cast<IO*>(split ? a.wv2 : nullptr), a.scale, a.cos_t, a.sin_t);
    GL_CHECK(hipGetLastError());
    t.launched();
  }
  {
    constexpr int rows_per_wg = kRedThreads / (D / 8);
    const dim3 grid(static_cast<unsigned>((a.total_tokens + rows_per_wg - 1) / rows_per_wg),
                    a.n_heads_kv);
    LaunchTiming t(tm, kKernReduce);
    auto fn = attn_bwd_reduce_kernel<IO, T, D, false>;
    if constexpr (sizeof(IO) == 2) {
      if (split) fn = attn_bwd_reduce_kernel<IO, T, D, true>;
    }
    GL_LAUNCH(t, fn, grid, dim3(kRedThreads), 0, st,
                          static_cast<const IO*>(a.wk), static_cast<const IO*>(a.wv),
                          a.single_seq ? nullptr : a.pos_of, a.cos_t, a.sin_t, a.total_tokens,
                          ratio, a.n_heads_kv, mfma32 && a.dkdv_head_pairs && ratio > 1 ? 2 : 1,
                          static_cast<IO*>(a.dk), static_cast<IO*>(a.dv),
                          static_cast<const IO*>(split ? a.wk2 : nullptr),
                          static_cast<const IO*>(split ? a.wv2 : nullptr),
                          split ? kTile * a.split : 0);
    GL_CHECK(hipGetLastError());
    t.launched();
  }
  return hipSuccess;
}

}  // namespace

// One instantiation per (tensor dtype, compute dtype, head_dim); fp32
// operands take head_dim up to 128 (a 256-wide fp32 K/V double buffer
// exceeds the LDS), bf16 operands up to 256.
template <template <typename, typename, int> class Impl, typename L>
hipError_t dispatch_head_dim(const L& a, hipStream_t st, KernelTimer* tm) {
  const bool bf = a.precision == kPrecBf16;
  switch (a.head_dim) {
#define GL_HEAD_DIM(DIM)                                                   \
  case DIM:                                                                \
    if (a.io_bf16) return Impl<bf16, bf16, DIM>::run(a, st, tm);          \
    if (bf) return Impl<float, bf16, DIM>::run(a, st, tm);                \
    if constexpr (DIM <= 128) return Impl<float, float, DIM>::run(a, st, tm); \
    return hipErrorInvalidValue;
    GL_HEAD_DIM(32)
    GL_HEAD_DIM(64)
    GL_HEAD_DIM(96)
    GL_HEAD_DIM(128)
    GL_HEAD_DIM(256)
#undef GL_HEAD_DIM
    default:
      return hipErrorInvalidValue;
  }
}

template <typename IO, typename T, int D>
struct ForwardImpl {
  static hipError_t run(const FwdLaunch& a, hipStream_t st, KernelTimer* tm) {
    return forward_impl<IO, T, D>(a, st, tm);
  }
};
template <typename IO, typename T, int D>
struct BackwardImpl {
  static hipError_t run(const BwdLaunch& a, hipStream_t st, KernelTimer* tm) {
    return backward_impl<IO, T, D>(a, st, tm);
  }
};

hipError_t launch_forward(const FwdLaunch& a, hipStream_t st, KernelTimer* tm) {
  return dispatch_head_dim<ForwardImpl>(a, st, tm);
}

hipError_t launch_backward(const BwdLaunch& a, hipStream_t st, KernelTimer* tm) {
  return dispatch_head_dim<BackwardImpl>(a, st, tm);
}

size_t compute_elem_size(int precision, bool io_bf16) {
  return (io_bf16 || precision == kPrecBf16) ? 2 : 4;
}

}  // namespace glacier

#ifdef GLACIER_PHASE_STAMPS
// Profiling builds only: copies the phase stamps to host memory.
extern "C" int glacier_attn_debug_stamps(void* host, size_t bytes) {
  return static_cast<int>(hipMemcpyFromSymbol(host, HIP_SYMBOL(glacier::glacier_stamps), bytes));
}
#endif
