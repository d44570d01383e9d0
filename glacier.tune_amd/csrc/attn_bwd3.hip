// attn_bwd3.hip -- the bf16-tensor attention backward on 32x32x16 MFMAs
// (gfx950, wave64) for long sequences: GpuLoraEngine.Backward.cs:354-412
// (the dq/ds and dk/dv kernels of tune_bwd.cu:598-717) and the inverse
// rope_batch of :452, on device tensors; the arithmetic of
// CausalAttentionKernel.cs:79-213.
//
// Two launches before the GQA head reduction (attn_bwd_reduce):
//   bwd3_stats  per (query head, token) the pair (-lse log2 e, D_i), with
//               D_i = dO_i . O_i (the softmax-gradient row term), [Hq][T].
//   attn_bwd3   one workgroup of 8 waves per entry of the 128-row tile table
//               (both kinds, longest expected first):
//     dK/dV tile  128 keys of one query head, or of two (heads 2p, 2p + 1
//                 walked in sequence into the same accumulators, one
//                 partial per pair).  Waves = 4 key quarters x 2
//                 roles, the two waves of a quarter on one SIMD.  The P wave
//                 keeps its 32 keys' K fragments and dV^T in AGPRs and forms
//                 S = Q K^T, P (masked) and dV^T += dO^T P; the dS wave keeps
//                 V and dK^T, forms dP = dO V^T, dS = P (dP - D) and
//                 dK^T += Q^T dS.  P crosses to the dS wave through LDS.
//                 32-query chunks of Q, dO and the row stats stream through
//                 a 4-slot ring by DMA, two chunks ahead.
//     dQ tile     128 queries of one query head.  Waves = 4 query quarters x
//                 2 key groups (even and odd 32-key chunks, each group with
//                 its own 4-slot ring of K and V).  A wave keeps its queries'
//                 Q and dO fragments and dQ^T in AGPRs, forms S^T and dP^T,
//                 then dQ^T += K^T dS^T; the groups' sums are added in group
//                 order on the store, with the scale and the inverse RoPE.
//
// Matrix-core layout, v_mfma_f32_32x32x16_bf16 (lane l, c = l % 32,
// h = l / 32): A[row c][k = 8h .. 8h + 7], B[k = 8h ..][col c], and the
// accumulator holds column c, rows 8 (e / 4) + 4 h + e % 4 for e = 0 .. 15.
// A lane's accumulators therefore belong to one column (one key of S, one
// query of S^T) and 16 rows; elements 8 s .. 8 s + 7 are exactly the k-slots
// of k-step s of the next product (rows 16 s + 4 h + 0..3 and
// 16 s + 8 + 4 h + 0..3), whose A operand comes from two ds_read_b64_tr_b16
// reads of the row-major LDS tile (4 consecutive rows of one column each).
//
// LDS tiles are [32][D] bf16 rows, unpadded, with 16-byte piece p of row r
// in slot p ^ lds_sw(r), which keeps both access patterns conflict-free: a
// 16-lane quarter of a fragment read (16 rows, one piece each) and a 32-lane
// half of a transposing read (4 rows x 4 pieces).
//
// Steps: every wave takes every step with one workgroup barrier.  Step c
// forms chunk c's first products (a dependent chain) and issues chunk
// c - 1's last products (independent MFMAs) between the chain's links; the
// ring slot of every LDS read is an immediate offset (the steady loop is
// unrolled over the four slots).
//
// All sums have a fixed order and no atomics are used: results are bitwise
// repeatable.
#include "attn_common.hpp"
#include "attn_ks.hpp"
#include "attn_launch.hpp"
#include "lds_mfma.hpp"

#include <hip/hip_ext.h>

namespace glacier {
namespace {


constexpr int kW3 = 8;
constexpr int kNT3 = kW3 * 64;
constexpr int kC3 = 32;  // rows per chunk

template <int D>
struct L3 {
  static constexpr int RB = 2 * D;        // bytes per bf16 row
  static constexpr int CB = kC3 * RB;     // bytes per 32-row chunk
  static constexpr int NKK = D / 16;      // k-steps over head_dim
  static constexpr int NDB = D / 32;      // 32-row blocks of head_dim
  static constexpr int ST = 256;          // stats bytes per chunk: 32 x (-lse log2 e), 32 x D
  static constexpr int SLOT = 2 * CB;     // one ring slot: Q + dO (dK/dV kind) or K + V (dQ)
  // dK/dV kind: the stats of the 4 ring slots, the ring, then per key
  // quarter two P hand-over areas (16 floats per lane each)
  static constexpr int KV_STATS = 4 * ST;
  static constexpr int KV_RING = 4 * SLOT;
  static constexpr int KV_BYTES = KV_STATS + KV_RING + 4 * 2 * 4096;
  // dQ kind: per key group a ring of 4 slots
  static constexpr int Q_BYTES = 2 * 4 * SLOT;
  // merge: every wave's accumulator (NDB x 16 floats per lane)
  static constexpr int REG = NDB * 16 * 64 * 4;
  static constexpr int MERGE = kW3 * REG;
  static constexpr int BYTES = KV_BYTES > Q_BYTES ? (KV_BYTES > MERGE ? KV_BYTES : MERGE)
                                                  : (Q_BYTES > MERGE ? Q_BYTES : MERGE);
  static_assert(BYTES <= 160 * 1024, "exceeds the LDS of a CU");
  // every LDS read's immediate offset fits the 16-bit field
  static_assert(KV_STATS + 3 * SLOT + CB + 16 * RB < 65536, "ring offsets");
};



// x += A B, x in VGPRs (read by VALU code after the chain), B resident in
// AGPRs.  The compiler sees no MFMA here; a chain's first product is
// mma32_zero (no accumulator input), later ones accumulate into the same
// registers back to back, which needs no wait states; xdl_to_valu() must
// separate the chain's last MFMA from any VALU read of x.
__device__ inline void mma32(f32x16& x, const bf16x8& a, const bf16x8& b) {
  asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+v"(x) : "v"(a), "a"(b));
}
// the wait states between a 16-pass MFMA's result and a VALU read of it
__device__ inline void xdl_to_valu(f32x16& x) {
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" : "+v"(x));
}
// acc += A B with the accumulator pinned in AGPRs (the compiler sees no
// MFMA, so the asm carries the wait states a VALU-written operand needs;
// back-to-back accumulation into the same registers needs none).
__device__ inline void mma32_acc(f32x16& acc, const bf16x8& a, const bf16x8& b) {
  asm volatile("s_nop 1\n\tv_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b));
}
template <int N>
__device__ inline void zero16(f32x16 (&a)[N]) {
  f32x16 z;
#pragma unroll
  for (int e = 0; e < 16; ++e) z[e] = 0.0f;
#pragma unroll
  for (int j = 0; j < N; ++j) asm volatile("" : "=a"(a[j]) : "0"(z));
}
template <int N>
__device__ inline void home16(f32x16 (&a)[N]) {
#pragma unroll
  for (int j = 0; j < N; ++j) asm volatile("" : "+a"(a[j]));
}
// the wait states an MFMA result needs before anything else reads it
template <int N>
__device__ inline void fence16(f32x16 (&a)[N]) {
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
#pragma unroll
  for (int j = 0; j < N; ++j) asm volatile("" : "+a"(a[j]));
}
__device__ inline void lds_w4(unsigned addr, const f32x4& v) {
  asm volatile("ds_write_b128 %0, %1" : : "v"(addr), "v"(v) : "memory");
}
// A wave's accumulators (AGPRs, after fence16) into its merge region: f32x4
// q of block db of lane l at byte (4 db + q) 1024 + 16 l of the region
// (base: region + 16 l).  The values pass through VGPRs, a block at a time.
template <int N>
__device__ inline void write_accs(unsigned base, const f32x16 (&acc)[N]) {
#pragma unroll
  for (int db = 0; db < N; ++db) {
    const f32x16 y = acc[db];
#pragma unroll
    for (int q = 0; q < 4; ++q)
      lds_w4(base + 1024u * (4 * db + q), f32x4{y[4 * q], y[4 * q + 1], y[4 * q + 2], y[4 * q + 3]});
  }
}

// ---- DMA into swizzled [32][D] tiles --------------------------------------
// Instruction n of a 32-row chunk fills LDS bytes 1024 n .. of the tile;
// lane l writes the 16 bytes at 16 l, i.e. slot l % PPR of row
// n RPI + l / PPR, and loads the global piece slot ^ lds_sw(row) of that row.
// lds_sw depends on the row only modulo 16 = RPI P, so the per-lane part of
// the offset repeats every P instructions: it is computed once per tile
// (off[]), and the row block n RPI goes into the scalar offset.
template <int D>
struct Dma3 {
  static constexpr int PPR = D / 8, RPI = 64 / PPR, NI = kC3 / RPI, P = D == 128 ? 4 : 2;
  int off[P];  // per-lane byte offsets inside a full chunk
  int stat;    // per-lane offset of the row-stats copy
  int rowb;    // row stride, bytes (wave-uniform)
};
template <int D>
__device__ inline Dma3<D> dma3_setup(int rowb, int lane) {
  using M = Dma3<D>;
  Dma3<D> d;
  d.rowb = rowb;
  const int rl = lane / M::PPR, slot = lane % M::PPR;
#pragma unroll
  for (int j = 0; j < M::P; ++j) d.off[j] = rl * rowb + 16 * (slot ^ lds_sw<D>(j * M::RPI + rl));
  d.stat = 8 * (lane & 31) + 4 * (lane >> 5);
  return d;
}

// 32 rows from src (row stride d.rowb) into the tile at dst; rows at or past
// nvalid arrive as zeros (they lie outside the buffer resource).  A full
// chunk takes the precomputed offsets; a partial one (the last chunk of a
// sequence) computes its offsets per lane.
template <int D>
__device__ inline void dma3(const Dma3<D>& d, const bf16* src, int nvalid, unsigned char* dst,
                            int lane) {
#if defined(__HIP_DEVICE_COMPILE__)
  using M = Dma3<D>;
  if (nvalid >= kC3) {
    const __amdgpu_buffer_rsrc_t rs = wave_rsrc(src, kC3 * d.rowb);
#pragma unroll
    for (int n = 0; n < M::NI; ++n)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (GLACIER_LDS void*)(dst + 1024 * n), 16,
                                               d.off[n % M::P], n * M::RPI * d.rowb, 0, 0);
  } else {
    const int nv = nvalid < 0 ? 0 : nvalid;
    const __amdgpu_buffer_rsrc_t rs = wave_rsrc(src, nv * d.rowb);
    const int ln = fresh_v(lane);
    const int rl = ln / M::PPR, slot = ln % M::PPR;
#pragma unroll
    for (int n = 0; n < M::NI; ++n) {
      const int r = n * M::RPI + rl;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (GLACIER_LDS void*)(dst + 1024 * n), 16,
                                               r * d.rowb + 16 * (slot ^ lds_sw<D>(r)), 0, 0, 0);
    }
  }
#endif
}

// The row stats of 32 queries (float2 (-lse log2 e, D) per query, from src)
// into a 256-byte LDS area, split: the first component of query i at byte
// 4 i, the second at 128 + 4 i.  Queries at or past nvalid arrive as zeros.
template <int D>
__device__ inline void dma_stats3(const Dma3<D>& d, const float2* src, int nvalid,
                                  unsigned char* dst) {
#if defined(__HIP_DEVICE_COMPILE__)
  const int nv = nvalid < 0 ? 0 : nvalid < kC3 ? nvalid : kC3;
  const __amdgpu_buffer_rsrc_t rs = wave_rsrc(src, nv * 8);
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (GLACIER_LDS void*)dst, 4, d.stat, 0, 0, 0);
#endif
}

// The B (or A) fragments of 32 rows held in registers: lane l takes row
// l % 32 at elements 16 kk + 8 (l / 32) .. + 7, for every k-step kk.  Rows
// at or past nvalid read as zeros.
template <int D>
__device__ inline void load_rows3(const bf16* src, int rowb, int nvalid, bf16x8 (&f)[D / 16],
                                  int lane) {
#if defined(__HIP_DEVICE_COMPILE__)
  const int nv = nvalid < 0 ? 0 : nvalid < kC3 ? nvalid : kC3;
  const __amdgpu_buffer_rsrc_t rs = wave_rsrc(src, nv * rowb);
  const int off = (lane & 31) * rowb + 16 * (lane >> 5);
#pragma unroll
  for (int kk = 0; kk < D / 16; ++kk)
    f[kk] = __builtin_bit_cast(bf16x8, __builtin_amdgcn_raw_buffer_load_b128(rs, off + 32 * kk, 0, 0));
#endif
}

// Byte offset of this lane's fragment read (row lane % 32, piece
// 2 kk + lane / 32) at k-step 0; k-step kk is that offset ^ 32 kk.
template <int D>
__device__ inline unsigned frag3(int lane) {
  const int r = lane & 31, h = lane >> 5;
  return static_cast<unsigned>(r * 2 * D + 16 * (h ^ lds_sw<D>(r)));
}
// Byte offset of this lane's transposing read for column block 0, row set
// t (rows 8 t + 4 h + 0..3 of the chunk's first 16); column block db is
// that offset ^ 64 db, rows 16 .. 31 at + 16 rows.
template <int D>
__device__ inline unsigned tr3(int lane, int t) {
  const int G = lane >> 4, i = lane & 15, h = lane >> 5;
  const int row = 8 * t + 4 * h + (i >> 2);
  const int col = 16 * (G & 1) + 4 * (i & 3);
  return static_cast<unsigned>(row * 2 * D + 16 * ((col >> 3) ^ lds_sw<D>(row)) + 2 * (col & 7));
}

// Every LDS read address a wave needs in its loop, computed once per tile:
// f[kk] the fragment read of k-step kk from a tile at fbase, t[db][j] the
// transposing reads of column block db (row sets j = 0, 1) from a tile at
// tbase.  The ring slot and the row block of a read enter as the immediate
// offset of the instruction.
template <int D>
struct Rd3 {
  unsigned f[D / 16];
  unsigned t[D / 32][2];
};
template <int D>
__device__ inline Rd3<D> rd3_setup(unsigned fbase, unsigned tbase, int lane) {
  Rd3<D> r;
  const unsigned fo = frag3<D>(lane), t0 = tr3<D>(lane, 0), t1 = tr3<D>(lane, 1);
#pragma unroll
  for (int kk = 0; kk < D / 16; ++kk) r.f[kk] = fbase + (fo ^ (32u * kk));
#pragma unroll
  for (int db = 0; db < D / 32; ++db) {
    r.t[db][0] = tbase + (t0 ^ (64u * db));
    r.t[db][1] = tbase + (t1 ^ (64u * db));
  }
  return r;
}

template <int OFF>
__device__ inline f32x4 lds4o(unsigned addr) {
  f32x4 r;
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "i"(OFF));
  return r;
}
template <int OFF>
__device__ inline void lds_w4o(unsigned addr, const f32x4& v) {
  asm volatile("ds_write_b128 %0, %1 offset:%2" : : "v"(addr), "v"(v), "i"(OFF) : "memory");
}
// x = A B (the first MFMA of a chain: the accumulator starts at zero)
__device__ inline void mma32_zero(f32x16& x, const bf16x8& a, const bf16x8& b) {
  asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, 0" : "=v"(x) : "v"(a), "a"(b));
}

// ---------------------------------------------------------------------------
// bwd3_stats: grid (tokens / rows per workgroup, query heads); one D/8-lane
// group per (token, head) row, each lane multiplying 8 elements of dO and O
// in order, the group adding the partials in a fixed order.  Writes
// (-lse log2 e, D_i) per (head, token).
// ---------------------------------------------------------------------------
template <int D>
__global__ __launch_bounds__(256) void bwd3_stats_kernel(const bf16* __restrict__ d_out,
                                                         const bf16* __restrict__ out,
                                                         const float* __restrict__ lse,
                                                         float2* __restrict__ stats,
                                                         int total_tokens, int n_heads_q) {
  constexpr int LPR = D / 8;
  constexpr int RPW = 256 / LPR;
  const int tok = blockIdx.x * RPW + threadIdx.x / LPR;
  const int h = blockIdx.y;
  const int part = threadIdx.x % LPR;
  const int tt = tok < total_tokens ? tok : total_tokens - 1;
  const long rr = (long)tt * n_heads_q + h;
  const long si = (long)h * total_tokens + tt;
  const float l = lse[si];
  float xd[8], xo[8];
  load8(d_out + rr * D + 8 * part, xd);
  load8(out + rr * D + 8 * part, xo);
  float acc = 0.0f;
#pragma unroll
  for (int e = 0; e < 8; ++e) acc += xd[e] * xo[e];
  const float drow = lanes_sum<LPR>(acc);
  if (tok < total_tokens && part == 0) stats[si] = make_float2(-l * kLog2e, drow);
}

// ---------------------------------------------------------------------------
// Steps.  Both tile kinds run one loop of steps with one workgroup barrier
// each; every wave takes every step (a chunk that lies entirely before a
// wave's keys, or after its queries, is computed fully masked: its
// contribution is exactly zero, and the wave would wait at the barrier
// anyway).  Chunk c of a ring lives in slot c % 4; at step c the chunk
// c + 2 is copied in by DMA (its slot held chunk c - 2, last read at step
// c - 1) and must have landed by the end of step c + 1.  Step c forms chunk
// c's first products (a dependent chain of 8 MFMAs) and issues chunk
// c - 1's last products (independent MFMAs) between the chain's links, so
// each link's latency is filled.  The ring position of every read is an
// immediate offset: the steady loop is unrolled over the four slots.
// ---------------------------------------------------------------------------

// ---------------------------------------------------------------------------
// dK/dV tile: 128 keys of one query head.  8 waves = 4 key quarters x 2
// roles; the two waves of a key quarter share a SIMD.  The P wave keeps its
// 32 keys' K fragments and dV^T in AGPRs: at step c it forms S(c) = Q K^T
// while accumulating dV^T += dO^T P(c - 1), then P(c) = exp2(S scale log2 e
// - lse log2 e) (masked), which it hands to its partner through LDS.  The
// dS wave keeps V and dK^T: at step c it forms dS(c - 1) = P(c - 1)
// (dP(c - 1) - D), then dP(c) = dO V^T while accumulating
// dK^T += Q^T dS(c - 1).  The P wave's exponentials end its step and the dS
// wave's arithmetic begins its step, so the two overlap on their SIMD.
// ---------------------------------------------------------------------------
template <int D>
__device__ inline void b4_dkdv(const TileDesc td, const bf16* __restrict__ q_rot,
                               const bf16* __restrict__ d_out, const bf16* __restrict__ k_rot,
                               const bf16* __restrict__ v, const float2* __restrict__ stats,
                               bf16* __restrict__ wk, bf16* __restrict__ wv, int total_tokens,
                               int n_heads_q, int n_heads_kv, int h, int hp, int kvh, float c2,
                               float scale, unsigned char* smem) {
  using L = L3<D>;
  constexpr int NKK = L::NKK, NDB = L::NDB, NST = 2 * NDB;
  constexpr int RING = L::KV_RING, SL = L::SLOT;
  const int w = wave_id(), lane = threadIdx.x & 63;
  GL_STAMP(kKernBwd, 0);
  GL_STAMP_VALUE(kKernBwd, 31, td.tile);
  const int kq = w & 3, role = w >> 2;
  const int k0 = kWideTile * td.tile;
  const int kw = k0 + 32 * kq;                          // this wave's first key
  const int nst = (td.len - k0 + kC3 - 1) / kC3;        // 32-query chunks from k0 on, per head
  // hp query heads (h, h + 1) in sequence: chunk n is chunk n % nst of head
  // h + n / nst; the accumulators run on across the heads
  const int ntot = hp * nst;
  auto local = [&](int n) { return n >= nst ? n - nst : n; };
  const long qstride = (long)n_heads_q * D, kvstride = (long)n_heads_kv * D;
  const int qrowb = static_cast<int>(qstride * 2), kvrowb = static_cast<int>(kvstride * 2);
  const bf16* qb0 = q_rot + ((long)td.tok0 * n_heads_q + h) * D;
  const bf16* ob0 = d_out + ((long)td.tok0 * n_heads_q + h) * D;
  const float2* sb0 = stats + (long)h * total_tokens + td.tok0;
  const unsigned sbase = static_cast<unsigned>(reinterpret_cast<uintptr_t>((GLACIER_LDS void*)smem));
  // this wave's reads: its own operand (Q for S, dO for dP) as fragments,
  // the other one transposed (dO^T for dV, Q^T for dK), its stats (-lse
  // log2 e or D), the hand-over area of its key quarter (two buffers)
  const unsigned ring = sbase + L::KV_STATS;
  const Rd3<D> rd = rd3_setup<D>(ring + (role == 0 ? 0u : static_cast<unsigned>(L::CB)),
                                 ring + (role == 0 ? static_cast<unsigned>(L::CB) : 0u), lane);
  const unsigned sta = sbase + (role == 0 ? 0u : 128u) + 16u * (lane >> 5);
  const unsigned hb = sbase + static_cast<unsigned>(L::KV_STATS + RING + kq * 8192) + 16u * lane;
  const Dma3<D> dq3 = dma3_setup<D>(qrowb, lane);
  // chunk n into its slot, by three dS waves: Q (key quarter 0), dO (1),
  // the stats (2)
  auto issue = [&](int n) {
    if (role != 1 || kq == 3) return;
    const int hh = n >= nst ? 1 : 0;
    const int q0 = k0 + kC3 * (n - hh * nst), sl = n & 3;
    if (kq == 0)
      dma3<D>(dq3, qb0 + hh * D + (long)q0 * qstride, td.len - q0, smem + L::KV_STATS + sl * SL, lane);
    else if (kq == 1)
      dma3<D>(dq3, ob0 + hh * D + (long)q0 * qstride, td.len - q0,
              smem + L::KV_STATS + sl * SL + L::CB, lane);
    else
      dma_stats3<D>(dq3, sb0 + (long)hh * total_tokens + q0, td.len - q0, smem + sl * L::ST);
  };
  // DMA instructions per chunk of this wave (for its waits)
  const int per = role == 1 ? (kq < 2 ? D / 16 : kq == 2 ? 1 : 0) : 0;
  auto mask_of = [&](int m) {
    // (m: the chunk's index within its head) the chunk's first query
    // precedes the wave's last key, or the chunk or the wave's keys run past
    // the sequence end
    return k0 + kC3 * m < kw + 31 || k0 + kC3 * (m + 1) > td.len || kw + 32 > td.len;
  };

  // Prologue: the wave's 32 K rows (P waves) or V rows (dS waves) into
  // AGPRs, chunks 0 and 1.
  bf16x8 kf[NKK];
  load_rows3<D>((role == 0 ? k_rot : v) + ((long)(td.tok0 + kw) * n_heads_kv + kvh) * D, kvrowb,
                td.len - kw, kf, lane);
  issue(0);
  if (ntot > 1) issue(1);
  f32x16 acc[NDB];
  zero16(acc);
  vmw<0>();
#pragma unroll
  for (int kk = 0; kk < NKK; ++kk) asm volatile("" : "+a"(kf[kk]));
  __syncthreads();
  GL_STAMP(kKernBwd, 1);

  // Wave state across steps: the B operands of chunk c - 1's products (P
  // waves: P(c - 1), formed at the end of step c - 1; dS waves: dS(c - 1),
  // formed at the start of step c), two sets by chunk parity; dS waves also
  // keep dP(c - 1) - D (two accumulators, by chunk parity).
  f32x16 xs[2];
  bf16x8 opb[2][2];

  // One step.  A: chunk c's chain (slot SA), B: chunk c - 1's products
  // (slot SB); HA, HB: whether the step has them; q0: chunk c's first query.
  auto step = [&](auto sa, auto sb, auto ha, auto hb_, int c) {
    constexpr int SA = decltype(sa)::value, SB = decltype(sb)::value;
    constexpr bool HA = decltype(ha)::value, HB = decltype(hb_)::value;
    constexpr int PA = SA & 1, PB = SB & 1;  // chunk parities (ring of 4)
    constexpr int OA = SA * SL, OB = SB * SL;
    // the dS wave first forms dS(c - 1) as bf16 B operands
    if constexpr (HB) {
      if (role == 1) {
        f32x4 pr[4];
        pr[0] = lds4o<PB * 4096 + 0>(hb);
        pr[1] = lds4o<PB * 4096 + 1024>(hb);
        pr[2] = lds4o<PB * 4096 + 2048>(hb);
        pr[3] = lds4o<PB * 4096 + 3072>(hb);
        lgkm<0>();
        f32x16& xp = xs[PB];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          tie_v(pr[j]);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float d = pr[j][e] * xp[4 * j + e];
            opb[PB][(4 * j + e) >> 3][(4 * j + e) & 7] = (bf16)d;
          }
        }
      }
    }
    // link j: fragment read kk = j of chunk c, transposing reads of step j
    // of chunk c - 1; reads run PF links ahead
    constexpr int NL = NKK > NST ? NKK : NST, PF = 4;
    bf16x8 fa[NKK];
    bf16x4 ta[NST][2];
    auto issue_link = [&](auto jc) {
      constexpr int j = decltype(jc)::value;
      if constexpr (HA && j < NKK) fa[j] = rd128<OA>(rd.f[j]);
      if constexpr (HB && j < NST) {
        ta[j][0] = rdtr<OB + 16 * (j & 1) * L::RB>(rd.t[j >> 1][0]);
        ta[j][1] = rdtr<OB + 16 * (j & 1) * L::RB>(rd.t[j >> 1][1]);
      }
    };
    constexpr int RPL = (HA ? 1 : 0) + (HB ? 2 : 0);  // reads per link
    static_for<PF>([&](auto jc) { issue_link(jc); });
    f32x16& xa = xs[PA];
    static_for<NL>([&](auto jc) {
      constexpr int j = decltype(jc)::value;
      constexpr int ahead = (NL - 1 - j) < (PF - 1) ? (NL - 1 - j) : (PF - 1);
      lgkm<RPL * ahead>();
      if constexpr (HA && j < NKK) {
        tie_v(fa[j]);
        if constexpr (j == 0)
          mma32_zero(xa, fa[j], kf[j]);
        else
          mma32(xa, fa[j], kf[j]);
      }
      if constexpr (HB && j < NST) {
        tie_v(ta[j][0]);
        tie_v(ta[j][1]);
        mma32_acc(acc[j >> 1], join8(ta[j][0], ta[j][1]), opb[PB][j & 1]);
      }
      if constexpr (j + PF < NL) issue_link(std::integral_constant<int, j + PF>{});
    });
    if constexpr (HA) {
      // stats of chunk c (the P wave's -lse log2 e, the dS wave's D), read
      // while the chain drains
      f32x4 st[4];
      st[0] = lds4o<SA * L::ST + 0>(sta);
      st[1] = lds4o<SA * L::ST + 32>(sta);
      st[2] = lds4o<SA * L::ST + 64>(sta);
      st[3] = lds4o<SA * L::ST + 96>(sta);
      xdl_to_valu(xa);
      lgkm<0>();
#pragma unroll
      for (int j = 0; j < 4; ++j) tie_v(st[j]);
      if (role == 0) {
        // P(c), masked, handed over and kept as bf16 for dV at step c + 1
#pragma unroll
        for (int e = 0; e < 16; ++e)
          xa[e] = __builtin_amdgcn_exp2f(__builtin_fmaf(xa[e], c2, st[e >> 2][e & 3]));
        const int cl = local(c);
        if (mask_of(cl)) {
          const int key = kw + (lane & 31), hh = lane >> 5, q0 = k0 + kC3 * cl;
#pragma unroll
          for (int e = 0; e < 16; ++e) {
            const int q = q0 + 8 * (e >> 2) + 4 * hh + (e & 3);
            if (!(key <= q && q < td.len)) xa[e] = 0.0f;
          }
        }
        lds_w4o<PA * 4096 + 0>(hb, f32x4{xa[0], xa[1], xa[2], xa[3]});
        lds_w4o<PA * 4096 + 1024>(hb, f32x4{xa[4], xa[5], xa[6], xa[7]});
        lds_w4o<PA * 4096 + 2048>(hb, f32x4{xa[8], xa[9], xa[10], xa[11]});
        lds_w4o<PA * 4096 + 3072>(hb, f32x4{xa[12], xa[13], xa[14], xa[15]});
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
#pragma unroll
          for (int j = 0; j < 8; ++j) opb[PA][ks][j] = (bf16)xa[8 * ks + j];
        lgkm<0>();
      } else {
#pragma unroll
        for (int e = 0; e < 16; ++e) xa[e] -= st[e >> 2][e & 3];
      }
    }
    // a step with no chain ends on its products: their wait states come
    // before any copy the compiler makes of the accumulators
    if constexpr (!HA) fence16(acc);
  };
  using B0 = std::false_type;
  using B1 = std::true_type;
  // DMA bookkeeping of step c: chunk c + 2 goes out at the start; chunk
  // c + 1 must have landed by the end (chunk c + 2's copy may stay in flight)
  auto dma_begin = [&](int c) {
    if (c + 2 < ntot) issue(c + 2);
  };
  auto dma_end = [&](int c) {
    if (per == 0) return;
    if (c + 2 < ntot)
      vm_wait_v(per);
    else
      vmw<0>();
  };
  // step 0: chain of chunk 0 only
  dma_begin(0);
  step(std::integral_constant<int, 0>{}, std::integral_constant<int, 3>{}, B1{}, B0{}, 0);
  dma_end(0);
  GL_STAMP(kKernBwd, 4);
  wg_barrier();
  // steps 1 .. ntot - 1: chains of chunk c, products of chunk c - 1, in
  // groups of four by slot
  int c = 1;
  auto full = [&](auto sa, int cc) {
    constexpr int SA = decltype(sa)::value;
    dma_begin(cc);
    step(sa, std::integral_constant<int, (SA + 3) & 3>{}, B1{}, B1{}, cc);
    dma_end(cc);
    if (cc < 12) GL_STAMP(kKernBwd, 4 + cc);
    wg_barrier();
  };
#pragma clang loop unroll(disable)
  for (; c + 3 < ntot; c += 4) {
    full(std::integral_constant<int, 1>{}, c);
    full(std::integral_constant<int, 2>{}, c + 1);
    full(std::integral_constant<int, 3>{}, c + 2);
    full(std::integral_constant<int, 0>{}, c + 3);
  }
  if (c < ntot) {
    full(std::integral_constant<int, 1>{}, c);
    ++c;
  }
  if (c < ntot) {
    full(std::integral_constant<int, 2>{}, c);
    ++c;
  }
  if (c < ntot) {
    full(std::integral_constant<int, 3>{}, c);
    ++c;
  }
  // step ntot: products of the last chunk only
  switch ((ntot - 1) & 3) {
    case 0: step(std::integral_constant<int, 1>{}, std::integral_constant<int, 0>{}, B0{}, B1{}, ntot); break;
    case 1: step(std::integral_constant<int, 2>{}, std::integral_constant<int, 1>{}, B0{}, B1{}, ntot); break;
    case 2: step(std::integral_constant<int, 3>{}, std::integral_constant<int, 2>{}, B0{}, B1{}, ntot); break;
    default: step(std::integral_constant<int, 0>{}, std::integral_constant<int, 3>{}, B0{}, B1{}, ntot); break;
  }
  GL_STAMP(kKernBwd, 20);

  fence16(acc);
  // Merge: every wave writes its accumulator into its region; then all
  // threads store the partials (dK scaled) as 4-element row pieces.
  __syncthreads();
  write_accs(sbase + static_cast<unsigned>(w * L::REG + lane * 16), acc);
  lgkm<0>();
  __syncthreads();
  {
    // slot (j4 = 4 db + qq, source lane sl) of region w holds elements
    // d = 32 db + 8 qq + 4 (sl / 32) .. + 3 of key sl % 32 of key quarter w % 4;
    // a thread's pieces are read in batches of eight, one wait per batch
    constexpr int NSLOT = 4 * NDB * 64;
    constexpr int NIT = kW3 * NSLOT / kNT3, NB = 8;
    static_assert(NIT % NB == 0, "epilogue batches");
#pragma unroll
    for (int b0 = 0; b0 < NIT; b0 += NB) {
      f32x4 a[NB];
#pragma unroll
      for (int t = 0; t < NB; ++t) {
        const int i2 = threadIdx.x + kNT3 * (b0 + t);
        a[t] = lds4(sbase + static_cast<unsigned>((i2 / NSLOT) * L::REG + (i2 % NSLOT) * 16));
      }
      lgkm<0>();
#pragma unroll
      for (int t = 0; t < NB; ++t) {
        tie_v(a[t]);
        const int i2 = threadIdx.x + kNT3 * (b0 + t);
        const int wr = i2 / NSLOT, j = i2 % NSLOT;
        const int kqr = wr & 3, rr = wr >> 2;
        const int j4 = j >> 6, sl = j & 63;
        const int db = j4 >> 2, qq = j4 & 3;
        const int key = k0 + 32 * kqr + (sl & 31);
        const int d0 = 32 * db + 8 * qq + 4 * (sl >> 5);
        bf16* dst = rr == 0 ? wv : wk;
        if (key < td.len)
          store4(dst + ((long)(td.tok0 + key) * n_heads_q + h) * D + d0, rr == 0 ? a[t] : a[t] * scale);
      }
    }
  }
  GL_STAMP(kKernBwd, 22);
}

// ---------------------------------------------------------------------------
// dQ tile: 128 queries of one query head.  8 waves = 4 query quarters x 2
// key groups (chunks kg, kg + 2, ... of the keys before the tile's end, each
// group through its own ring).  A wave keeps its 32 queries' Q and dO
// fragments (the B operands of S^T = K Q^T and dP^T = V dO^T) and dQ^T in
// AGPRs.  At step c it forms S^T(c) and dP^T(c) (two chains, linked
// alternately) while accumulating dQ^T += K^T dS^T(c - 1), then
// dS^T(c) = P (dP - D) as bf16 B operands for step c + 1.
// ---------------------------------------------------------------------------
template <int D>
__device__ inline void b4_dq(const TileDesc td, const bf16* __restrict__ q_rot,
                             const bf16* __restrict__ d_out, const bf16* __restrict__ k_rot,
                             const bf16* __restrict__ v, const float2* __restrict__ stats,
                             bf16* __restrict__ dq, const int32_t* __restrict__ pos_of,
                             int total_tokens, int n_heads_q, int n_heads_kv, int h, int kvh,
                             float c2, float scale, const float* __restrict__ cos_t,
                             const float* __restrict__ sin_t, unsigned char* smem) {
  using L = L3<D>;
  constexpr int NKK = L::NKK, NDB = L::NDB, NST = 2 * NDB, H = D / 2;
  constexpr int SL = L::SLOT;
  const int w = wave_id(), lane = threadIdx.x & 63;
  GL_STAMP(kKernBwd, 0);
  GL_STAMP_VALUE(kKernBwd, 31, 100 + td.tile);
  const int qq = w & 3, kg = w >> 2;
  const int q0t = kWideTile * td.tile;
  const int qw = q0t + 32 * qq;                       // this wave's first query
  const int kend = min(td.len, q0t + kWideTile);      // keys before this (the causal range)
  const int nks = (kend + kC3 - 1) / kC3;             // 32-key chunks
  const int nch = (nks + 1) / 2;                      // steps with a chunk (group 0 has the most)
  const int mych = (nks - kg + 1) / 2;                // this group's chunks
  const long qstride = (long)n_heads_q * D, kvstride = (long)n_heads_kv * D;
  const int qrowb = static_cast<int>(qstride * 2), kvrowb = static_cast<int>(kvstride * 2);
  const bf16* kb0 = k_rot + ((long)td.tok0 * n_heads_kv + kvh) * D;
  const bf16* vb0 = v + ((long)td.tok0 * n_heads_kv + kvh) * D;
  const unsigned sbase = static_cast<unsigned>(reinterpret_cast<uintptr_t>((GLACIER_LDS void*)smem));
  const unsigned gbase = sbase + static_cast<unsigned>(kg * 4 * SL);
  const Rd3<D> rd = rd3_setup<D>(gbase, gbase, lane);  // K fragments (V at + CB), K transposed
  const Dma3<D> dk3 = dma3_setup<D>(kvrowb, lane);
  // this group's chunk i (keys 32 (kg + 2 i) ..) into slot i % 4: K by query
  // quarter 0, V by query quarter 1
  auto issue = [&](int i) {
    if (qq > 1 || i >= mych) return;
    const int r0 = kC3 * (kg + 2 * i);
    unsigned char* dst = smem + kg * 4 * SL + (i & 3) * SL;
    if (qq == 0)
      dma3<D>(dk3, kb0 + (long)r0 * kvstride, td.len - r0, dst, lane);
    else
      dma3<D>(dk3, vb0 + (long)r0 * kvstride, td.len - r0, dst + L::CB, lane);
  };
  const int per = qq < 2 ? D / 16 : 0;

  // Prologue: this wave's Q and dO rows into AGPRs, its query's row stats
  // (rows past the sequence end are computed but never stored), chunks 0, 1.
  bf16x8 qf[NKK], of[NKK];
  load_rows3<D>(q_rot + ((long)(td.tok0 + qw) * n_heads_q + h) * D, qrowb, td.len - qw, qf, lane);
  load_rows3<D>(d_out + ((long)(td.tok0 + qw) * n_heads_q + h) * D, qrowb, td.len - qw, of, lane);
  const int qi = min(qw + (lane & 31), td.len - 1);
  const float2 stq = stats[(long)h * total_tokens + td.tok0 + qi];
  issue(0);
  issue(1);
  f32x16 acc[NDB];
  zero16(acc);
  vmw<0>();
#pragma unroll
  for (int kk = 0; kk < NKK; ++kk) {
    asm volatile("" : "+a"(qf[kk]));
    asm volatile("" : "+a"(of[kk]));
  }
  const float nl = stq.x, dd = stq.y;
  __syncthreads();
  GL_STAMP(kKernBwd, 1);

  bf16x8 dsb[2][2];  // dS^T(c) as bf16 B operands, by chunk parity
  auto step = [&](auto sa, auto sb, auto ha, auto hb_, int c) {
    constexpr int SA = decltype(sa)::value, SB = decltype(sb)::value;
    constexpr bool HA = decltype(ha)::value, HB = decltype(hb_)::value;
    constexpr int PA = SA & 1, PB = SB & 1;
    constexpr int OA = SA * SL, OB = SB * SL;
    constexpr int NL = NKK > NST ? NKK : NST, PF = 3;
    constexpr int RPL = (HA ? 2 : 0) + (HB ? 2 : 0);
    bf16x8 fk[NKK], fv[NKK];
    bf16x4 ta[NST][2];
    auto issue_link = [&](auto jc) {
      constexpr int j = decltype(jc)::value;
      if constexpr (HA && j < NKK) {
        fk[j] = rd128<OA>(rd.f[j]);
        fv[j] = rd128<OA + L::CB>(rd.f[j]);
      }
      if constexpr (HB && j < NST) {
        ta[j][0] = rdtr<OB + 16 * (j & 1) * L::RB>(rd.t[j >> 1][0]);
        ta[j][1] = rdtr<OB + 16 * (j & 1) * L::RB>(rd.t[j >> 1][1]);
      }
    };
    static_for<PF>([&](auto jc) { issue_link(jc); });
    f32x16 s, dp;
    static_for<NL>([&](auto jc) {
      constexpr int j = decltype(jc)::value;
      constexpr int ahead = (NL - 1 - j) < (PF - 1) ? (NL - 1 - j) : (PF - 1);
      lgkm<RPL * ahead>();
      if constexpr (HA && j < NKK) {
        tie_v(fk[j]);
        tie_v(fv[j]);
        if constexpr (j == 0) {
          mma32_zero(s, fk[j], qf[j]);
          mma32_zero(dp, fv[j], of[j]);
        } else {
          mma32(s, fk[j], qf[j]);
          mma32(dp, fv[j], of[j]);
        }
      }
      if constexpr (HB && j < NST) {
        tie_v(ta[j][0]);
        tie_v(ta[j][1]);
        mma32_acc(acc[j >> 1], join8(ta[j][0], ta[j][1]), dsb[PB][j & 1]);
      }
      if constexpr (j + PF < NL) issue_link(std::integral_constant<int, j + PF>{});
    });
    if constexpr (HA) {
      xdl_to_valu(s);
      xdl_to_valu(dp);
      const int m = kg + 2 * c;  // chunk c's key chunk
      float d[16];
#pragma unroll
      for (int e = 0; e < 16; ++e)
        d[e] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[e], c2, nl)) * (dp[e] - dd);
      if (kC3 * m + 31 > qw) {  // keys past the wave's first query: the causal mask
        const int q = qw + (lane & 31), hh = lane >> 5;
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int key = kC3 * m + 8 * (e >> 2) + 4 * hh + (e & 3);
          if (key > q) d[e] = 0.0f;
        }
      }
#pragma unroll
      for (int ks = 0; ks < 2; ++ks)
#pragma unroll
        for (int j = 0; j < 8; ++j) dsb[PA][ks][j] = (bf16)d[8 * ks + j];
    }
    if constexpr (!HA) fence16(acc);
  };
  using B0 = std::false_type;
  using B1 = std::true_type;
  auto dma_begin = [&](int c) { issue(c + 2); };
  auto dma_end = [&](int c) {
    if (per == 0) return;
    if (c + 2 < mych)
      vm_wait_v(per);
    else
      vmw<0>();
  };
  // a group with fewer chunks than group 0 runs its last step as an empty
  // chain: the chunk slots past its end hold no DMA, so its step is B-only
  int c = 0;
  if (mych > 0) {
    dma_begin(0);
    step(std::integral_constant<int, 0>{}, std::integral_constant<int, 3>{}, B1{}, B0{}, 0);
    dma_end(0);
  }
  GL_STAMP(kKernBwd, 4);
  wg_barrier();
  c = 1;
  auto full = [&](auto sa, int cc) {
    constexpr int SA = decltype(sa)::value;
    dma_begin(cc);
    step(sa, std::integral_constant<int, (SA + 3) & 3>{}, B1{}, B1{}, cc);
    dma_end(cc);
    if (cc < 12) GL_STAMP(kKernBwd, 4 + cc);
    wg_barrier();
  };
#pragma clang loop unroll(disable)
  for (; c + 3 < mych; c += 4) {
    full(std::integral_constant<int, 1>{}, c);
    full(std::integral_constant<int, 2>{}, c + 1);
    full(std::integral_constant<int, 3>{}, c + 2);
    full(std::integral_constant<int, 0>{}, c + 3);
  }
  if (c < mych) {
    full(std::integral_constant<int, 1>{}, c);
    ++c;
  }
  if (c < mych) {
    full(std::integral_constant<int, 2>{}, c);
    ++c;
  }
  if (c < mych) {
    full(std::integral_constant<int, 3>{}, c);
    ++c;
  }
  // the last chunk's products, then the barriers group 0 still has
  if (mych > 0) {
    switch ((mych - 1) & 3) {
      case 0: step(std::integral_constant<int, 1>{}, std::integral_constant<int, 0>{}, B0{}, B1{}, mych); break;
      case 1: step(std::integral_constant<int, 2>{}, std::integral_constant<int, 1>{}, B0{}, B1{}, mych); break;
      case 2: step(std::integral_constant<int, 3>{}, std::integral_constant<int, 2>{}, B0{}, B1{}, mych); break;
      default: step(std::integral_constant<int, 0>{}, std::integral_constant<int, 3>{}, B0{}, B1{}, mych); break;
    }
  }
  // every wave passes 1 + nch barriers in the loop above (a group with
  // mych chunks passes 1 + max(mych - 1, 0)); make up the difference
  for (int k = (mych > 0 ? mych : 1); k < nch; ++k) wg_barrier();
  GL_STAMP(kKernBwd, 20);

  // Merge: every wave writes its sums into region (key group, query
  // quarter); then all threads add the two key groups of each element in
  // group order, scale, apply the inverse RoPE at the query's position and
  // store rows of dq.  A thread takes elements d0 .. d0 + 3 and d0 + D/2 ..
  // (the rotation pairs: column block db and db + NDB/2 of one slot) of one
  // query, NIT such pieces; their cos/sin are loaded first, so that those
  // loads (and the position lookups before them) run beside the merge.
  constexpr int NHALF = 2 * NDB * 64;  // slots of column blocks 0 .. NDB/2 - 1
  constexpr int NIT = 4 * NHALF / kNT3;
  static_assert(NIT * kNT3 == 4 * NHALF, "epilogue pieces");
  f32x4 pcs[NIT], psn[NIT];
#pragma unroll
  for (int it = 0; it < NIT; ++it) {
    const int i2 = threadIdx.x + kNT3 * it;
    const int qqr = i2 / NHALF, j = i2 % NHALF;
    const int j4 = j >> 6, sl = j & 63;
    const int db = j4 >> 2, qp = j4 & 3;
    const int qi2 = min(q0t + 32 * qqr + (sl & 31), td.len - 1);
    const int d0 = 32 * db + 8 * qp + 4 * (sl >> 5);
    const long pos = pos_of != nullptr ? pos_of[td.tok0 + qi2] : qi2;
    pcs[it] = *reinterpret_cast<const f32x4*>(cos_t + pos * H + d0);
    psn[it] = *reinterpret_cast<const f32x4*>(sin_t + pos * H + d0);
  }
  fence16(acc);
  __syncthreads();
  write_accs(sbase + static_cast<unsigned>((kg * 4 + qq) * L::REG + lane * 16), acc);
  lgkm<0>();
  __syncthreads();
#pragma unroll
  for (int it = 0; it < NIT; ++it) {
    const int i2 = threadIdx.x + kNT3 * it;
    const int qqr = i2 / NHALF, j = i2 % NHALF;
    const int j4 = j >> 6, sl = j & 63;
    const int db = j4 >> 2, qp = j4 & 3;
    const unsigned off0 = static_cast<unsigned>(j * 16);
    const unsigned off1 = off0 + (NDB / 2) * 4 * 1024;  // column block db + NDB / 2
    f32x4 lo0 = lds4(sbase + static_cast<unsigned>(qqr * L::REG) + off0);
    f32x4 hi0 = lds4(sbase + static_cast<unsigned>(qqr * L::REG) + off1);
    f32x4 lo1 = lds4(sbase + static_cast<unsigned>((4 + qqr) * L::REG) + off0);
    f32x4 hi1 = lds4(sbase + static_cast<unsigned>((4 + qqr) * L::REG) + off1);
    lgkm<0>();
    tie_v(lo0);
    tie_v(hi0);
    tie_v(lo1);
    tie_v(hi1);
    lo0 += lo1;
    hi0 += hi1;
    const int qi2 = q0t + 32 * qqr + (sl & 31);
    const int d0 = 32 * db + 8 * qp + 4 * (sl >> 5);  // elements d0 .. d0 + 3 and H + d0 ..
    if (qi2 < td.len) {
      const f32x4 cs = pcs[it], sn = psn[it];
      const f32x4 a = lo0 * scale, b = hi0 * scale;
      f32x4 y0, y1;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        float u0, u1;
        rope_inv(a[r], b[r], cs[r], sn[r], u0, u1);
        y0[r] = u0;
        y1[r] = u1;
      }
      bf16* row_p = dq + ((long)(td.tok0 + qi2) * n_heads_q + h) * D;
      store4(row_p + d0, y0);
      store4(row_p + H + d0, y1);
    }
  }
  GL_STAMP(kKernBwd, 22);
}

// grid (ratio, Hkv, entries) or, with head_pairs, (ceil(ratio / 2), Hkv,
// entries) (ratio = Hq / Hkv); z indexes the tile table (both kinds,
// longest expected first).  head_pairs: x stands for query heads 2x and
// 2x + 1 of the group (the last one alone when ratio is odd): a dK/dV tile
// walks both heads' queries into the same accumulators (one partial per
// pair); the table then holds each dQ tile twice, kTileDq for head 2x and
// kTileDqSecond for head 2x + 1.
// The arguments needed first lead (preloaded in SGPRs: build.py).
template <int D>
__global__ __launch_bounds__(kNT3) void attn_bwd3_kernel(
    const TileDesc* __restrict__ tiles_bwd, int ratio, int head_pairs, int total_tokens, float c2,
    const bf16* __restrict__ q_rot, const bf16* __restrict__ d_out, const bf16* __restrict__ k_rot,
    const bf16* __restrict__ v, const float2* __restrict__ stats, bf16* __restrict__ dq,
    bf16* __restrict__ wk, bf16* __restrict__ wv, const int32_t* __restrict__ pos_of, float scale,
    const float* __restrict__ cos_t, const float* __restrict__ sin_t) {
  extern __shared__ __align__(16) unsigned char smem_raw[];
  const int n_heads_kv = gridDim.y, n_heads_q = ratio * n_heads_kv;
  // Head pairs: the x index is rotated so that with an odd group the pair
  // holding one head (half a dK/dV tile's work, no second dQ tile) falls to
  // every dispatch queue in turn.  The hardware deals workgroup ids to the 8
  // XCDs and, within each, to its 4 shader engines in turn: id mod 32 fixes
  // the 8 CUs that run a workgroup.  An odd group rotates by the id's round
  // of 32 (rotated by the entry index, a queue saw the entries of one parity
  // only, i.e. two of the four pairs of a 7-head group, and the engines'
  // loads differed by a quarter: S=4096 backward 434 -> 417 us with the
  // round); an even group, whose pairs cost the same, keeps the entry index
  // (0.6% faster at Llama-3 B=2 S=2048).  Either rotation is the same for
  // all x of one (y, z), so it permutes the pairs.
  const int rot = (ratio & 1) ? static_cast<int>((gridDim.x * (blockIdx.z * gridDim.y + blockIdx.y)) >> 5)
                              : static_cast<int>(blockIdx.z);
  const int x = head_pairs ? 2 * (((int)blockIdx.x + rot) % (int)gridDim.x) : (int)blockIdx.x;
  const int kvh = blockIdx.y;
  const TileDesc td = tiles_bwd[blockIdx.z];
  if (td.kind == kTileDkDv) {
    const int hp = head_pairs && ratio - x >= 2 ? 2 : 1;
    b4_dkdv<D>(td, q_rot, d_out, k_rot, v, stats, wk, wv, total_tokens, n_heads_q, n_heads_kv,
               kvh * ratio + x, hp, kvh, c2, scale, smem_raw);
  } else {
    const int hq = x + (td.kind == kTileDqSecond ? 1 : 0);
    if (hq >= ratio) return;  // an odd group's last pair has no second head
    b4_dq<D>(td, q_rot, d_out, k_rot, v, stats, dq, pos_of, total_tokens, n_heads_q, n_heads_kv,
             kvh * ratio + hq, kvh, c2, scale, cos_t, sin_t, smem_raw);
  }
#ifdef GLACIER_PHASE_STAMPS
  // profiling builds: the workgroup's end is its last wave's (slot 22 is
  // wave 0's)
  __syncthreads();
  GL_STAMP(kKernBwd, 25);
  // where it ran: HW_ID (CU, shader array, engine) and XCC_ID
  GL_STAMP_VALUE(kKernBwd, 26, __builtin_amdgcn_s_getreg((31 << 11) | 4));
  GL_STAMP_VALUE(kKernBwd, 27, __builtin_amdgcn_s_getreg((31 << 11) | 20));
#endif
}

}  // namespace

template <int D>
hipError_t launch_bwd3(const BwdLaunch& a, hipStream_t st, KernelTimer* tm) {
  const int ratio = a.n_heads_q / a.n_heads_kv;
  float2* stats = static_cast<float2*>(a.stats);
  {
    constexpr int rows_per_wg = 256 / (D / 8);
    const dim3 grid(static_cast<unsigned>((a.total_tokens + rows_per_wg - 1) / rows_per_wg),
                    a.n_heads_q);
    LaunchTiming t(tm, kKernBwdStats);
    GL_LAUNCH(t, (bwd3_stats_kernel<D>), grid, dim3(256), 0, st,
              static_cast<const bf16*>(a.d_out), static_cast<const bf16*>(a.out), a.lse, stats,
              a.total_tokens, a.n_heads_q);
    GL_CHECK(hipGetLastError());
    t.launched();
  }
  {
    auto fn = attn_bwd3_kernel<D>;
    constexpr size_t lds = L3<D>::BYTES;
    GL_CHECK(allow_lds(fn, lds));
    LaunchTiming t(tm, kKernBwd);
    const bool pairs = a.dkdv_head_pairs && ratio > 1;
    GL_LAUNCH(t, fn, dim3(pairs ? (ratio + 1) / 2 : ratio, a.n_heads_kv, a.n_wide_entries), dim3(kNT3),
              lds, st, a.tiles_wide, ratio, pairs ? 1 : 0, a.total_tokens, a.scale * kLog2e,
              static_cast<const bf16*>(a.q_rot), static_cast<const bf16*>(a.d_out),
              static_cast<const bf16*>(a.k_rot), static_cast<const bf16*>(a.v),
              static_cast<const float2*>(stats), static_cast<bf16*>(a.dq),
              static_cast<bf16*>(a.wk), static_cast<bf16*>(a.wv),
              a.single_seq ? nullptr : a.pos_of, a.scale, a.cos_t, a.sin_t);
    GL_CHECK(hipGetLastError());
    t.launched();
  }
  return hipSuccess;
}

template hipError_t launch_bwd3<64>(const BwdLaunch&, hipStream_t, KernelTimer*);
template hipError_t launch_bwd3<128>(const BwdLaunch&, hipStream_t, KernelTimer*);

}  // namespace glacier

#ifdef GLACIER_PHASE_STAMPS
// Profiling builds only: copies this file's phase stamps (the 32x32x16
// backward's) to host memory.
extern "C" int glacier_attn_debug_stamps_bwd3(void* host, size_t bytes) {
  return static_cast<int>(hipMemcpyFromSymbol(host, HIP_SYMBOL(glacier::glacier_stamps), bytes));
}
#endif
