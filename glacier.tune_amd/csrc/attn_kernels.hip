// attn_kernels.hip -- gfx950 kernels of the causal GQA attention path.
//
// Forward  (GpuLoraEngine.Forward.cs:401-465 rope_batch + tune_attn_causal_gqa_fwd):
//   kv_prep   K -> RoPE -> Kc (compute dtype, token-major) [+ k_rot out],
//             V -> Vt (compute dtype, [Hkv][D][padded tokens]).
//   attn_fwd  one workgroup = 64 queries of one head; 4 waves x 16 queries.
//             Q is rotated in registers on load (q_rot written if asked),
//             K and V^T tiles of 64 keys are staged in LDS and shared by the
//             4 waves; online softmax in fp32 (exp2 domain); O and the row
//             log-sum-exp are written at the end.  No [S,S] matrix exists.
// Backward (GpuLoraEngine.Backward.cs:354-412 dq_ds + dk_dv, :452 inverse rope):
//   bwd_prep  D_i = dO_i . O_i, transposed copies Q^T, dO^T, K^T (and
//             compute-dtype copies when the device tensors are fp32 and the
//             matrix cores run bf16).
//   attn_dq   one workgroup = 64 queries of one head: recomputes P from the
//             saved lse, dS = P (dP - D), dQ = scale * dS K, inverse RoPE.
//   attn_dkdv one workgroup = 64 keys of one (query head): dV_h = P^T dO,
//             dK_h = scale * dS^T Q accumulated in registers over all query
//             tiles, written as this head's partial (fp32).
//   dkdv_reduce  dK/dV = sum of the partials over the heads of the KV group
//             in ascending head order (the reference's lock-free workspace
//             reduction, CausalAttentionKernel.cs:184-206), inverse RoPE on dK.
// Every reduction has a fixed order and no kernel uses floating-point
// atomics, so results are bitwise repeatable (the activation-checkpoint
// recompute relies on that).
#include "attn_common.hpp"
#include "attn_launch.hpp"

namespace glacier {

// ---------------------------------------------------------------------------
// RoPE, written without contraction so that q_rot/k_rot are the exact fp32
// results of RoPEKernel.cs:84-85 (v0*c - v1*s, v0*s + v1*c) given the same
// cos/sin table.
// ---------------------------------------------------------------------------
__device__ inline void rope_fwd(float x0, float x1, float c, float s, float& y0,
                                float& y1) {
#pragma clang fp contract(off)
  y0 = x0 * c - x1 * s;
  y1 = x0 * s + x1 * c;
}
// inverse rotation (sin negated, RoPEKernel.cs:60)
__device__ inline void rope_inv(float x0, float x1, float c, float s, float& y0,
                                float& y1) {
#pragma clang fp contract(off)
  y0 = x0 * c + x1 * s;
  y1 = x1 * c - x0 * s;
}

__device__ inline void load8(const float* p, float (&x)[8]) {
  float4 a = *reinterpret_cast<const float4*>(p);
  float4 b = *reinterpret_cast<const float4*>(p + 4);
  x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w;
  x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
}
__device__ inline void load8(const bf16* p, float (&x)[8]) {
  bf16x8 v = *reinterpret_cast<const bf16x8*>(p);
#pragma unroll
  for (int i = 0; i < 8; ++i) x[i] = (float)v[i];
}
__device__ inline void store8(float* p, const float (&x)[8]) {
  *reinterpret_cast<float4*>(p) = make_float4(x[0], x[1], x[2], x[3]);
  *reinterpret_cast<float4*>(p + 4) = make_float4(x[4], x[5], x[6], x[7]);
}
__device__ inline void store8(bf16* p, const float (&x)[8]) {
  bf16x8 v;
#pragma unroll
  for (int i = 0; i < 8; ++i) v[i] = (bf16)x[i];
  *reinterpret_cast<bf16x8*>(p) = v;
}
__device__ inline void store4(float* p, f32x4 v) {
  *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
}
__device__ inline void store4(bf16* p, f32x4 v) {
  bf16x4 b;
#pragma unroll
  for (int i = 0; i < 4; ++i) b[i] = (bf16)v[i];
  *reinterpret_cast<bf16x4*>(p) = b;
}

// Global (token-major) fragment of row `row` for k-step kk.
template <typename T>
__device__ inline typename Mfma<T>::Frag frag_global(const T* rowp, int kk, int g) {
  using M = Mfma<T>;
  const T* p = rowp + kk * M::KSTEP + M::KPL * g;
  if constexpr (sizeof(T) == 2) {
    return *reinterpret_cast<const bf16x8*>(p);
  } else {
    return *p;
  }
}

template <typename T>
__device__ inline typename Mfma<T>::Frag frag_zero() {
  if constexpr (sizeof(T) == 2) {
    bf16x8 z;
#pragma unroll
    for (int i = 0; i < 8; ++i) z[i] = (bf16)0.0f;
    return z;
  } else {
    return 0.0f;
  }
}

// ---------------------------------------------------------------------------
// Copy one [64 rows][D] block (rows r < nvalid of src, row stride gstride)
// into a transposed destination dst[d * dstride + r] (64 columns, zeros for
// r >= nvalid) and, if dst_rm is given, a row-major compute-dtype copy.
// `lds` holds 64 * (D + 2) elements of T.
// ---------------------------------------------------------------------------
template <typename IO, typename T, int D>
__device__ inline void transpose_block(const IO* src, long gstride, int nvalid,
                                       T* dst_tr, long dstride, T* dst_rm,
                                       long rm_stride, T* lds, int tid) {
  constexpr int LS = D + 2;
  // phase 1: rows -> LDS (8 consecutive elements per thread and step)
  constexpr int CPR = D / 8;
  for (int idx = tid; idx < kTile * CPR; idx += kThreads) {
    int r = idx / CPR, ch = idx % CPR;
    float x[8];
    if (r < nvalid) {
      load8(src + (long)r * gstride + ch * 8, x);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) x[e] = 0.0f;
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) lds[r * LS + ch * 8 + e] = from_f32<T>(x[e]);
    if (dst_rm != nullptr && r < nvalid) store8(dst_rm + (long)r * rm_stride + ch * 8, x);
  }
  __syncthreads();
  // phase 2: LDS columns -> transposed rows (16-byte chunks)
  constexpr int CE = 16 / sizeof(T);
  constexpr int CPT = kTile / CE;
  for (int idx = tid; idx < D * CPT; idx += kThreads) {
    int d = idx / CPT, ch = idx % CPT;
    union {
      uint4 u;
      T e[CE];
    } pk;
#pragma unroll
    for (int e = 0; e < CE; ++e) pk.e[e] = lds[(ch * CE + e) * LS + d];
    *reinterpret_cast<uint4*>(dst_tr + (long)d * dstride + ch * CE) = pk.u;
  }
}

// ---------------------------------------------------------------------------
// kv_prep: grid (Hkv, ntiles).
// ---------------------------------------------------------------------------
template <typename IO, typename T, int D>
__global__ __launch_bounds__(kThreads) void kv_prep_kernel(
    const IO* __restrict__ k, const IO* __restrict__ v, T* __restrict__ kc,
    IO* __restrict__ k_rot, T* __restrict__ vt, const TileDesc* __restrict__ tiles,
    int n_heads_kv, int ptot, const float* __restrict__ cos_t,
    const float* __restrict__ sin_t) {
  __shared__ T lds[kTile * (D + 2)];
  const int j = blockIdx.x;
  const TileDesc td = tiles[blockIdx.y];
  const int tid = threadIdx.x;
  const int row0 = kTile * td.tile;
  const int nvalid = min(kTile, td.len - row0);
  constexpr int H = D / 2;
  // K: rotate each pair (p, p + D/2) of each valid row.
  for (int idx = tid; idx < kTile * H; idx += kThreads) {
    int r = idx / H, p = idx % H;
    if (r >= nvalid) continue;
    int pos = row0 + r;
    long base = ((long)(td.tok0 + pos) * n_heads_kv + j) * D;
    float x0 = to_f32(k[base + p]), x1 = to_f32(k[base + p + H]);
    float c = cos_t[(long)pos * H + p], s = sin_t[(long)pos * H + p];
    float y0, y1;
    rope_fwd(x0, x1, c, s, y0, y1);
    kc[base + p] = from_f32<T>(y0);
    kc[base + p + H] = from_f32<T>(y1);
    if (k_rot != nullptr) {
      k_rot[base + p] = from_f32<IO>(y0);
      k_rot[base + p + H] = from_f32<IO>(y1);
    }
  }
  // V -> V^T (zero columns past the sequence end)
  transpose_block<IO, T, D>(v + ((long)td.tok0 * n_heads_kv + j) * D + (long)row0 * n_heads_kv * D,
                            (long)n_heads_kv * D, nvalid,
                            vt + (long)j * D * ptot + td.ptok0 + row0, ptot,
                            nullptr, 0, lds, tid);
}

// ---------------------------------------------------------------------------
// attn_fwd: grid (Hq, ntiles), 256 threads, dynamic LDS = K tile + V^T tile.
// ---------------------------------------------------------------------------
template <typename IO, typename T, int D>
__global__ __launch_bounds__(kThreads) void attn_fwd_kernel(
    const IO* __restrict__ q, const T* __restrict__ kc, const T* __restrict__ vt,
    IO* __restrict__ out, float* __restrict__ lse, IO* __restrict__ q_rot,
    const TileDesc* __restrict__ tiles, int n_heads_q, int n_heads_kv,
    int total_tokens, int ptot, float scale_log2, const float* __restrict__ cos_t,
    const float* __restrict__ sin_t) {
  using M = Mfma<T>;
  using L = Lds<T, D>;
  constexpr int NKD = D / M::KSTEP;
  constexpr int H = D / 2;
  extern __shared__ __align__(16) unsigned char smem_raw[];
  T* ks = reinterpret_cast<T*>(smem_raw);
  T* vts = ks + L::RM_ELEMS;

  const int h = blockIdx.x;
  const TileDesc td = tiles[blockIdx.y];
  const int kvh = h / (n_heads_q / n_heads_kv);
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  const int g = lane >> 4, c = lane & 15;
  const int qrow = kTile * td.tile + 16 * w + c;
  const bool qvalid = qrow < td.len;
  const long qbase = ((long)(td.tok0 + qrow) * n_heads_q + h) * D;

  // Q fragments, rotated in fp32 then rounded to the compute dtype.
  typename M::Frag qf[NKD];
#pragma unroll
  for (int kk = 0; kk < NKD / 2; ++kk) {
    if constexpr (sizeof(T) == 2) {
      const int d0 = kk * M::KSTEP + 8 * g;
      float x0[8], x1[8], y0[8], y1[8];
      if (qvalid) {
        load8(q + qbase + d0, x0);
        load8(q + qbase + d0 + H, x1);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) x0[e] = x1[e] = 0.0f;
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const long ti = (long)(qvalid ? qrow : 0) * H + d0 + e;
        rope_fwd(x0[e], x1[e], cos_t[ti], sin_t[ti], y0[e], y1[e]);
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

  f32x4 o[D / 16];
#pragma unroll
  for (int db = 0; db < D / 16; ++db) o[db] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  float m_run = kNegBig, l_lane = 0.0f;

  const T* kbase = kc + ((long)td.tok0 * n_heads_kv + kvh) * D;
  const T* vtbase = vt + (long)kvh * D * ptot + td.ptok0;
  for (int kt = 0; kt <= td.tile; ++kt) {
    __syncthreads();
    stage_rm<T, D>(ks, kbase + (long)kTile * kt * n_heads_kv * D,
                   (long)n_heads_kv * D, td.len - kTile * kt, tid);
    stage_tr<T, D>(vts, vtbase + kTile * kt, ptot, tid);
    __syncthreads();

    const int nb = (kt == td.tile) ? (w + 1) : 4;
    float p[4][4];
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
        const int key = kTile * kt + 16 * b + 4 * g + r;
        const float t = (b < nb && key <= qrow) ? acc[r] * scale_log2 : -INFINITY;
        p[b][r] = t;
        mloc = fmaxf(mloc, t);
      }
    }
    mloc = col_max(mloc);
    const float m_new = fmaxf(m_run, mloc);
    const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
    float psum = 0.0f;
#pragma unroll
    for (int b = 0; b < 4; ++b)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        p[b][r] = __builtin_amdgcn_exp2f(p[b][r] - m_new);
        psum += p[b][r];
      }
    l_lane = l_lane * alpha + psum;
    m_run = m_new;
#pragma unroll
    for (int db = 0; db < D / 16; ++db) o[db] *= alpha;
    acc_tr<T, D>(o, vts, p, nb, lane);
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
// bwd_prep: grid (Hq + Hkv, ntiles).
// ---------------------------------------------------------------------------
template <typename IO, typename T, int D>
__global__ __launch_bounds__(kThreads) void bwd_prep_kernel(
    const IO* __restrict__ d_out, const IO* __restrict__ out,
    const IO* __restrict__ q_rot, const IO* __restrict__ k_rot,
    const IO* __restrict__ v, float* __restrict__ dvec, T* __restrict__ dot_t,
    T* __restrict__ qt, T* __restrict__ kt, T* __restrict__ doc,
    T* __restrict__ qc, T* __restrict__ kc, T* __restrict__ vc,
    const TileDesc* __restrict__ tiles, int n_heads_q, int n_heads_kv,
    int total_tokens, int ptot) {
  __shared__ T lds[kTile * (D + 2)];
  const int y = blockIdx.x;
  const TileDesc td = tiles[blockIdx.y];
  const int tid = threadIdx.x;
  const int row0 = kTile * td.tile;
  const int nvalid = min(kTile, td.len - row0);
  if (y < n_heads_q) {
    const int h = y;
    const long off = ((long)(td.tok0 + row0) * n_heads_q + h) * D;
    const long gs = (long)n_heads_q * D;
    // D_i = sum_d dO_i[d] * O_i[d]: 4 threads per row, fixed combine order.
    {
      const int r = tid >> 2, part = tid & 3;
      float acc = 0.0f;
      if (r < nvalid) {
        const IO* a = d_out + off + (long)r * gs + part * (D / 4);
        const IO* b = out + off + (long)r * gs + part * (D / 4);
        for (int d = 0; d < D / 4; d += 8) {
          float xa[8], xb[8];
          load8(a + d, xa);
          load8(b + d, xb);
#pragma unroll
          for (int e = 0; e < 8; ++e) acc += xa[e] * xb[e];
        }
      }
      acc += __shfl_xor(acc, 1);
      acc += __shfl_xor(acc, 2);
      if (r < nvalid && part == 0)
        dvec[(long)h * total_tokens + td.tok0 + row0 + r] = acc;
    }
    transpose_block<IO, T, D>(d_out + off, gs, nvalid,
                              dot_t + (long)h * D * ptot + td.ptok0 + row0, ptot,
                              doc != nullptr ? doc + off : nullptr, gs, lds, tid);
    __syncthreads();
    transpose_block<IO, T, D>(q_rot + off, gs, nvalid,
                              qt + (long)h * D * ptot + td.ptok0 + row0, ptot,
                              qc != nullptr ? qc + off : nullptr, gs, lds, tid);
  } else {
    const int j = y - n_heads_q;
    const long off = ((long)(td.tok0 + row0) * n_heads_kv + j) * D;
    const long gs = (long)n_heads_kv * D;
    transpose_block<IO, T, D>(k_rot + off, gs, nvalid,
                              kt + (long)j * D * ptot + td.ptok0 + row0, ptot,
                              kc != nullptr ? kc + off : nullptr, gs, lds, tid);
    if (vc != nullptr) {
      constexpr int CPR = D / 8;
      for (int idx = tid; idx < kTile * CPR; idx += kThreads) {
        int r = idx / CPR, ch = idx % CPR;
        if (r >= nvalid) continue;
        float x[8];
        load8(v + off + (long)r * gs + ch * 8, x);
        store8(vc + off + (long)r * gs + ch * 8, x);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// attn_dq: grid (Hq, ntiles), dynamic LDS = K tile + V tile + K^T tile.
// ---------------------------------------------------------------------------
template <typename IO, typename T, int D>
__global__ __launch_bounds__(kThreads) void attn_dq_kernel(
    const T* __restrict__ qsrc, const T* __restrict__ dosrc,
    const T* __restrict__ ksrc, const T* __restrict__ vsrc,
    const T* __restrict__ kt_g, const float* __restrict__ lse,
    const float* __restrict__ dvec, IO* __restrict__ dq,
    const TileDesc* __restrict__ tiles, int n_heads_q, int n_heads_kv,
    int total_tokens, int ptot, float scale_log2, float scale,
    const float* __restrict__ cos_t, const float* __restrict__ sin_t) {
  using M = Mfma<T>;
  using L = Lds<T, D>;
  constexpr int NKD = D / M::KSTEP;
  constexpr int H = D / 2;
  extern __shared__ __align__(16) unsigned char smem_raw[];
  T* ks = reinterpret_cast<T*>(smem_raw);
  T* vs = ks + L::RM_ELEMS;
  T* kts = vs + L::RM_ELEMS;

  const int h = blockIdx.x;
  const TileDesc td = tiles[blockIdx.y];
  const int kvh = h / (n_heads_q / n_heads_kv);
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  const int g = lane >> 4, c = lane & 15;
  const int qrow = kTile * td.tile + 16 * w + c;
  const bool qvalid = qrow < td.len;
  const long qbase = ((long)(td.tok0 + qrow) * n_heads_q + h) * D;

  typename M::Frag qf[NKD], df[NKD];
#pragma unroll
  for (int kk = 0; kk < NKD; ++kk) {
    qf[kk] = qvalid ? frag_global<T>(qsrc + qbase, kk, g) : frag_zero<T>();
    df[kk] = qvalid ? frag_global<T>(dosrc + qbase, kk, g) : frag_zero<T>();
  }
  const long si = (long)h * total_tokens + td.tok0 + qrow;
  const float lse2 = qvalid ? lse[si] * kLog2e : 0.0f;
  const float drow = qvalid ? dvec[si] : 0.0f;

  f32x4 acc_dq[D / 16];
#pragma unroll
  for (int db = 0; db < D / 16; ++db) acc_dq[db] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  const T* kb = ksrc + ((long)td.tok0 * n_heads_kv + kvh) * D;
  const T* vb = vsrc + ((long)td.tok0 * n_heads_kv + kvh) * D;
  const T* ktb = kt_g + (long)kvh * D * ptot + td.ptok0;
  for (int kt = 0; kt <= td.tile; ++kt) {
    __syncthreads();
    const long roff = (long)kTile * kt * n_heads_kv * D;
    stage_rm<T, D>(ks, kb + roff, (long)n_heads_kv * D, td.len - kTile * kt, tid);
    stage_rm<T, D>(vs, vb + roff, (long)n_heads_kv * D, td.len - kTile * kt, tid);
    stage_tr<T, D>(kts, ktb + kTile * kt, ptot, tid);
    __syncthreads();

    const int nb = (kt == td.tile) ? (w + 1) : 4;
    float ds[4][4];
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      f32x4 s = {0.0f, 0.0f, 0.0f, 0.0f}, dp = {0.0f, 0.0f, 0.0f, 0.0f};
      if (b < nb) {
#pragma unroll
        for (int kk = 0; kk < NKD; ++kk) {
          s = M::mma(frag_rm<T, D>(ks, 16 * b + c, kk, g), qf[kk], s);
          dp = M::mma(frag_rm<T, D>(vs, 16 * b + c, kk, g), df[kk], dp);
        }
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int key = kTile * kt + 16 * b + 4 * g + r;
        const bool ok = b < nb && key <= qrow;
        const float pv = ok ? __builtin_amdgcn_exp2f(s[r] * scale_log2 - lse2) : 0.0f;
        ds[b][r] = ok ? pv * (dp[r] - drow) : 0.0f;
      }
    }
    acc_tr<T, D>(acc_dq, kts, ds, nb, lane);
  }

  if (qvalid) {
#pragma unroll
    for (int db = 0; db < D / 32; ++db) {
      f32x4 lo = acc_dq[db] * scale, hi = acc_dq[db + D / 32] * scale;
      f32x4 y0, y1;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int d = 16 * db + 4 * g + r;
        const long ti = (long)qrow * H + d;
        float a, b;
        rope_inv(lo[r], hi[r], cos_t[ti], sin_t[ti], a, b);
        y0[r] = a;
        y1[r] = b;
      }
      store4(dq + qbase + 16 * db + 4 * g, y0);
      store4(dq + qbase + H + 16 * db + 4 * g, y1);
    }
  }
}

// ---------------------------------------------------------------------------
// attn_dkdv: grid (Hq, ntiles in key order); dynamic LDS = Q, dO tiles,
// Q^T, dO^T tiles, 64 lse and 64 D values.
// ---------------------------------------------------------------------------
template <typename T, int D>
__global__ __launch_bounds__(kThreads) void attn_dkdv_kernel(
    const T* __restrict__ qsrc, const T* __restrict__ dosrc,
    const T* __restrict__ ksrc, const T* __restrict__ vsrc,
    const T* __restrict__ qt_g, const T* __restrict__ dot_g,
    const float* __restrict__ lse, const float* __restrict__ dvec,
    float* __restrict__ wk, float* __restrict__ wv,
    const TileDesc* __restrict__ tiles, int n_heads_q, int n_heads_kv,
    int total_tokens, int ptot, float scale_log2, float scale) {
  using M = Mfma<T>;
  using L = Lds<T, D>;
  constexpr int NKD = D / M::KSTEP;
  extern __shared__ __align__(16) unsigned char smem_raw[];
  T* qs = reinterpret_cast<T*>(smem_raw);
  T* dos = qs + L::RM_ELEMS;
  T* qts = dos + L::RM_ELEMS;
  T* dots = qts + L::TR_ELEMS;
  float* lse_s = reinterpret_cast<float*>(dots + L::TR_ELEMS);
  float* d_s = lse_s + kTile;

  const int h = blockIdx.x;
  const TileDesc td = tiles[blockIdx.y];
  const int kvh = h / (n_heads_q / n_heads_kv);
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  const int g = lane >> 4, c = lane & 15;
  const int krow = kTile * td.tile + 16 * w + c;
  const bool kvalid = krow < td.len;
  const long kbase = ((long)(td.tok0 + krow) * n_heads_kv + kvh) * D;

  typename M::Frag kf[NKD], vf[NKD];
#pragma unroll
  for (int kk = 0; kk < NKD; ++kk) {
    kf[kk] = kvalid ? frag_global<T>(ksrc + kbase, kk, g) : frag_zero<T>();
    vf[kk] = kvalid ? frag_global<T>(vsrc + kbase, kk, g) : frag_zero<T>();
  }

  f32x4 acc_dk[D / 16], acc_dv[D / 16];
#pragma unroll
  for (int db = 0; db < D / 16; ++db) {
    acc_dk[db] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    acc_dv[db] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  }

  const int ntq = (td.len + kTile - 1) / kTile;
  const T* qb = qsrc + ((long)td.tok0 * n_heads_q + h) * D;
  const T* dob = dosrc + ((long)td.tok0 * n_heads_q + h) * D;
  const T* qtb = qt_g + (long)h * D * ptot + td.ptok0;
  const T* dotb = dot_g + (long)h * D * ptot + td.ptok0;
  const float* lseb = lse + (long)h * total_tokens + td.tok0;
  const float* db_ = dvec + (long)h * total_tokens + td.tok0;
  for (int qt = td.tile; qt < ntq; ++qt) {
    __syncthreads();
    const long roff = (long)kTile * qt * n_heads_q * D;
    const int nv = td.len - kTile * qt;
    stage_rm<T, D>(qs, qb + roff, (long)n_heads_q * D, nv, tid);
    stage_rm<T, D>(dos, dob + roff, (long)n_heads_q * D, nv, tid);
    stage_tr<T, D>(qts, qtb + kTile * qt, ptot, tid);
    stage_tr<T, D>(dots, dotb + kTile * qt, ptot, tid);
    if (tid < kTile) {
      const bool ok = tid < nv;
      lse_s[tid] = ok ? lseb[kTile * qt + tid] * kLog2e : 0.0f;
      d_s[tid] = ok ? db_[kTile * qt + tid] : 0.0f;
    }
    __syncthreads();

    const int b0 = (qt == td.tile) ? w : 0;  // query blocks below b0 are masked
    float p[4][4], ds[4][4];
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      f32x4 s = {0.0f, 0.0f, 0.0f, 0.0f}, dp = {0.0f, 0.0f, 0.0f, 0.0f};
      if (b >= b0) {
#pragma unroll
        for (int kk = 0; kk < NKD; ++kk) {
          s = M::mma(frag_rm<T, D>(qs, 16 * b + c, kk, g), kf[kk], s);
          dp = M::mma(frag_rm<T, D>(dos, 16 * b + c, kk, g), vf[kk], dp);
        }
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int qi = 16 * b + 4 * g + r;
        const int qrow = kTile * qt + qi;
        const bool ok = b >= b0 && krow <= qrow && qrow < td.len;
        const float pv = ok ? __builtin_amdgcn_exp2f(s[r] * scale_log2 - lse_s[qi]) : 0.0f;
        p[b][r] = pv;
        ds[b][r] = ok ? pv * (dp[r] - d_s[qi]) : 0.0f;
      }
    }
    acc_tr<T, D>(acc_dv, dots, p, 4, lane);
    acc_tr<T, D>(acc_dk, qts, ds, 4, lane);
  }

  if (kvalid) {
    const long wb = ((long)(td.tok0 + krow) * n_heads_q + h) * D;
#pragma unroll
    for (int db = 0; db < D / 16; ++db) {
      store4(wk + wb + 16 * db + 4 * g, acc_dk[db] * scale);
      store4(wv + wb + 16 * db + 4 * g, acc_dv[db]);
    }
  }
}

// ---------------------------------------------------------------------------
// dkdv_reduce: one thread per (token, kv head, pair p < D/2).
// ---------------------------------------------------------------------------
template <typename IO, int D>
__global__ __launch_bounds__(kThreads) void dkdv_reduce_kernel(
    const float* __restrict__ wk, const float* __restrict__ wv,
    IO* __restrict__ dk, IO* __restrict__ dv, const int32_t* __restrict__ pos_of,
    int total_tokens, int n_heads_q, int n_heads_kv,
    const float* __restrict__ cos_t, const float* __restrict__ sin_t) {
  constexpr int H = D / 2;
  const long idx = (long)blockIdx.x * kThreads + threadIdx.x;
  const long n = (long)total_tokens * n_heads_kv * H;
  if (idx >= n) return;
  const int p = idx % H;
  const int j = (idx / H) % n_heads_kv;
  const long tok = idx / ((long)H * n_heads_kv);
  const int ratio = n_heads_q / n_heads_kv;
  float k0 = 0.0f, k1 = 0.0f, v0 = 0.0f, v1 = 0.0f;
  for (int hh = 0; hh < ratio; ++hh) {
    const long src = (tok * n_heads_q + (long)j * ratio + hh) * D;
    k0 += wk[src + p];
    k1 += wk[src + p + H];
    v0 += wv[src + p];
    v1 += wv[src + p + H];
  }
  const int pos = pos_of[tok];
  float y0, y1;
  rope_inv(k0, k1, cos_t[(long)pos * H + p], sin_t[(long)pos * H + p], y0, y1);
  const long dst = (tok * n_heads_kv + j) * D;
  dk[dst + p] = from_f32<IO>(y0);
  dk[dst + p + H] = from_f32<IO>(y1);
  dv[dst + p] = from_f32<IO>(v0);
  dv[dst + p + H] = from_f32<IO>(v1);
}

// ---------------------------------------------------------------------------
// Host launchers
// ---------------------------------------------------------------------------
namespace {

template <typename T, int D>
constexpr size_t fwd_lds() {
  return sizeof(T) * (Lds<T, D>::RM_ELEMS + Lds<T, D>::TR_ELEMS);
}
template <typename T, int D>
constexpr size_t dq_lds() {
  return sizeof(T) * (2 * Lds<T, D>::RM_ELEMS + Lds<T, D>::TR_ELEMS);
}
template <typename T, int D>
constexpr size_t dkdv_lds() {
  return sizeof(T) * (2 * Lds<T, D>::RM_ELEMS + 2 * Lds<T, D>::TR_ELEMS) +
         2 * kTile * sizeof(float);
}

template <typename F>
hipError_t allow_lds(F* fn, size_t bytes) {
  if (bytes <= 65536) return hipSuccess;
  return hipFuncSetAttribute(reinterpret_cast<const void*>(fn),
                             hipFuncAttributeMaxDynamicSharedMemorySize,
                             static_cast<int>(bytes));
}

#define GL_CHECK(expr)                       \
  do {                                       \
    hipError_t e_ = (expr);                  \
    if (e_ != hipSuccess) return e_;         \
  } while (0)

template <typename IO, typename T, int D>
hipError_t forward_impl(const FwdLaunch& a, hipStream_t st, KernelTimer* tm) {
  const dim3 blk(kThreads);
  {
    ScopedTiming t(tm, kKernKvPrep, st);
    hipLaunchKernelGGL((kv_prep_kernel<IO, T, D>), dim3(a.n_heads_kv, a.n_tiles), blk, 0, st,
                       static_cast<const IO*>(a.k), static_cast<const IO*>(a.v),
                       static_cast<T*>(a.kc), static_cast<IO*>(a.k_rot),
                       static_cast<T*>(a.vt), a.tiles_any, a.n_heads_kv, a.ptot,
                       a.cos_t, a.sin_t);
    GL_CHECK(hipGetLastError());
  }
  {
    auto fn = attn_fwd_kernel<IO, T, D>;
    constexpr size_t lds = fwd_lds<T, D>();
    GL_CHECK(allow_lds(fn, lds));
    ScopedTiming t(tm, kKernFwd, st);
    hipLaunchKernelGGL(fn, dim3(a.n_heads_q, a.n_tiles), blk, lds, st,
                       static_cast<const IO*>(a.q), static_cast<const T*>(a.kc),
                       static_cast<const T*>(a.vt), static_cast<IO*>(a.out), a.lse,
                       static_cast<IO*>(a.q_rot), a.tiles_fwd, a.n_heads_q,
                       a.n_heads_kv, a.total_tokens, a.ptot, a.scale_log2,
                       a.cos_t, a.sin_t);
    GL_CHECK(hipGetLastError());
  }
  return hipSuccess;
}

template <typename IO, typename T, int D>
hipError_t backward_impl(const BwdLaunch& a, hipStream_t st, KernelTimer* tm) {
  const dim3 blk(kThreads);
  const bool same = std::is_same<IO, T>::value;
  {
    ScopedTiming t(tm, kKernBwdPrep, st);
    hipLaunchKernelGGL((bwd_prep_kernel<IO, T, D>),
                       dim3(a.n_heads_q + a.n_heads_kv, a.n_tiles), blk, 0, st,
                       static_cast<const IO*>(a.d_out), static_cast<const IO*>(a.out),
                       static_cast<const IO*>(a.q_rot), static_cast<const IO*>(a.k_rot),
                       static_cast<const IO*>(a.v), a.dvec, static_cast<T*>(a.dot_t),
                       static_cast<T*>(a.qt), static_cast<T*>(a.kt),
                       same ? nullptr : static_cast<T*>(a.doc),
                       same ? nullptr : static_cast<T*>(a.qc),
                       same ? nullptr : static_cast<T*>(a.kc),
                       same ? nullptr : static_cast<T*>(a.vc), a.tiles_any,
                       a.n_heads_q, a.n_heads_kv, a.total_tokens, a.ptot);
    GL_CHECK(hipGetLastError());
  }
  const T* qsrc = static_cast<const T*>(same ? a.q_rot : a.qc);
  const T* dosrc = static_cast<const T*>(same ? a.d_out : a.doc);
  const T* ksrc = static_cast<const T*>(same ? a.k_rot : a.kc);
  const T* vsrc = static_cast<const T*>(same ? a.v : a.vc);
  {
    auto fn = attn_dq_kernel<IO, T, D>;
    constexpr size_t lds = dq_lds<T, D>();
    GL_CHECK(allow_lds(fn, lds));
    ScopedTiming t(tm, kKernDq, st);
    hipLaunchKernelGGL(fn, dim3(a.n_heads_q, a.n_tiles), blk, lds, st, qsrc, dosrc,
                       ksrc, vsrc, static_cast<const T*>(a.kt), a.lse, a.dvec,
                       static_cast<IO*>(a.dq), a.tiles_fwd, a.n_heads_q,
                       a.n_heads_kv, a.total_tokens, a.ptot, a.scale_log2,
                       a.scale, a.cos_t, a.sin_t);
    GL_CHECK(hipGetLastError());
  }
  {
    auto fn = attn_dkdv_kernel<T, D>;
    constexpr size_t lds = dkdv_lds<T, D>();
    GL_CHECK(allow_lds(fn, lds));
    ScopedTiming t(tm, kKernDkdv, st);
    hipLaunchKernelGGL(fn, dim3(a.n_heads_q, a.n_tiles), blk, lds, st, qsrc, dosrc,
                       ksrc, vsrc, static_cast<const T*>(a.qt),
                       static_cast<const T*>(a.dot_t), a.lse, a.dvec, a.wk, a.wv,
                       a.tiles_kv, a.n_heads_q, a.n_heads_kv, a.total_tokens,
                       a.ptot, a.scale_log2, a.scale);
    GL_CHECK(hipGetLastError());
  }
  {
    const long n = (long)a.total_tokens * a.n_heads_kv * (D / 2);
    const unsigned grid = static_cast<unsigned>((n + kThreads - 1) / kThreads);
    ScopedTiming t(tm, kKernReduce, st);
    hipLaunchKernelGGL((dkdv_reduce_kernel<IO, D>), dim3(grid), blk, 0, st, a.wk, a.wv,
                       static_cast<IO*>(a.dk), static_cast<IO*>(a.dv), a.pos_of,
                       a.total_tokens, a.n_heads_q, a.n_heads_kv, a.cos_t, a.sin_t);
    GL_CHECK(hipGetLastError());
  }
  return hipSuccess;
}

}  // namespace

hipError_t launch_forward(const FwdLaunch& a, hipStream_t st, KernelTimer* tm) {
  const bool bf = a.precision == kPrecBf16;
  if (a.io_bf16) {
    if (a.head_dim == 64) return forward_impl<bf16, bf16, 64>(a, st, tm);
    return forward_impl<bf16, bf16, 128>(a, st, tm);
  }
  if (bf) {
    if (a.head_dim == 64) return forward_impl<float, bf16, 64>(a, st, tm);
    return forward_impl<float, bf16, 128>(a, st, tm);
  }
  if (a.head_dim == 64) return forward_impl<float, float, 64>(a, st, tm);
  return forward_impl<float, float, 128>(a, st, tm);
}

hipError_t launch_backward(const BwdLaunch& a, hipStream_t st, KernelTimer* tm) {
  const bool bf = a.precision == kPrecBf16;
  if (a.io_bf16) {
    if (a.head_dim == 64) return backward_impl<bf16, bf16, 64>(a, st, tm);
    return backward_impl<bf16, bf16, 128>(a, st, tm);
  }
  if (bf) {
    if (a.head_dim == 64) return backward_impl<float, bf16, 64>(a, st, tm);
    return backward_impl<float, bf16, 128>(a, st, tm);
  }
  if (a.head_dim == 64) return backward_impl<float, float, 64>(a, st, tm);
  return backward_impl<float, float, 128>(a, st, tm);
}

size_t compute_elem_size(int precision, bool io_bf16) {
  return (io_bf16 || precision == kPrecBf16) ? 2 : 4;
}

}  // namespace glacier
