// attn_bwd.hip -- the bf16-MFMA attention backward for bf16 tensors (gfx950,
// wave64): GpuLoraEngine.Backward.cs:354-412 (tune_attn_causal_gqa_bwd_dq_ds
// and _bwd_dk_dv) and the inverse rope_batch of :452, on device tensors.
//
// Two launches before the GQA head reduction (attn_bwd_reduce, attn_kernels.hip):
//   bwd_stats  per (query head, token): -lse * log2(e) and the softmax-gradient
//              row term D_i = dO_i . O_i, as one float2 [Hq][T] array.
//   attn_bwd2  one workgroup of 8 waves per tile; the tile table mixes two
//              kinds, longest expected first:
//     dK/dV tile  64 keys of one query head.  Waves = 2 key halves x 4
//                 query groups; a wave owns 32 keys (two 16-key MFMA blocks,
//                 so every fragment it reads from LDS feeds two MFMAs), and
//                 group g takes the 32-query stages g, g + 4, ... of the
//                 causal range.  S = Q K^T and dP = dO V^T with the keys as
//                 MFMA columns, P from the row stats, dS = P (dP - D);
//                 dV^T += dO^T P and dK^T += Q^T dS accumulate in registers;
//                 the four groups' sums are added in group order and written
//                 as this head's partial (bf16 rows).
//     dQ tile     64 queries of one query head.  Waves = 2 query halves x 4
//                 key groups; a wave owns 32 queries and group g takes the
//                 32-key stages g, g + 4, ...; S^T = K Q^T and dP^T = V dO^T
//                 with the queries as columns, dQ^T += K^T dS^T; the groups'
//                 sums are added in group order, scaled, inverse-rotated and
//                 written as rows of dq.
// Every streamed stage goes from L2 into XOR-swizzled LDS tiles by DMA
// (buffer_load ... lds), one stage ahead, with one workgroup barrier per
// stage; LDS reads are issued from inline assembly with explicit waits (the
// compiler would tie its own forms to every outstanding DMA).  All sums have
// a fixed order and no atomics are used: results are bitwise repeatable.
#include "attn_common.hpp"
#include "attn_ks.hpp"
#include "attn_launch.hpp"

#include <hip/hip_ext.h>

#include <utility>

namespace glacier {
namespace {

constexpr int kB2Waves = 8;
constexpr int kB2Threads = kB2Waves * 64;
constexpr int kGroups = 4;  // stage groups (2 waves each)

template <int D>
struct B2Layout {
  static constexpr int CB = kChunk * D * 2;      // bytes of one 32-row bf16 chunk
  // dK/dV kind: the tile's 64 K rows and 64 V rows, then per group two slots
  // of (Q, dO) (the row stats are read from global memory)
  static constexpr int KTILE = 2 * CB;
  static constexpr int VTILE = KTILE;
  static constexpr int SLOT_KV = 2 * CB;
  static constexpr int KV_BYTES = KTILE + VTILE + 2 * kGroups * SLOT_KV;
  // dQ kind: per group two slots of (K, V)
  static constexpr int SLOT_Q = 2 * CB;
  static constexpr int Q_BYTES = 2 * kGroups * SLOT_Q;
  static constexpr int BYTES = KV_BYTES > Q_BYTES ? KV_BYTES : Q_BYTES;
  static_assert(BYTES <= 160 * 1024, "exceeds the LDS of a CU");
  // group merge: 8 waves x (one tensor's accumulators: 2 (D/16) f32x4 per lane)
  static constexpr int MERGE = 8 * 2 * (D / 16) * 64 * 16;
  static_assert(MERGE <= BYTES, "merge area exceeds the LDS");
};

// ---- LDS reads from inline assembly (see attn_ks.hpp) -------------------
template <int OFF>
__device__ inline f32x4 lds_f4(unsigned addr) {
  f32x4 r;
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "i"(OFF));
  return r;
}
__device__ inline void lgkm_wait0() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }
// at most N LDS reads of this wave still outstanding (they complete in order)
template <int N>
__device__ inline void lgkm_wait() {
  static_assert(N >= 0 && N < 16, "lgkmcnt range");
  asm volatile("s_waitcnt lgkmcnt(%0)" ::"i"(N) : "memory");
}
// lgkm_wait with a count known only after unrolling (a multiple of 2, < 16)
__device__ inline void lgkm_wait_n(int n) {
  switch (n) {
    case 0: lgkm_wait<0>(); break;
    case 2: lgkm_wait<2>(); break;
    case 4: lgkm_wait<4>(); break;
    case 6: lgkm_wait<6>(); break;
    case 8: lgkm_wait<8>(); break;
    case 10: lgkm_wait<10>(); break;
    case 12: lgkm_wait<12>(); break;
    default: lgkm_wait<0>(); break;
  }
}
template <typename T>
__device__ inline void tie(T& x) {
  asm volatile("" : "+v"(x));
}
// A copy of x that the compiler must treat as new at this point: values
// derived from it inside a loop body (LDS addresses, mask indices: one VALU
// operation each) are recomputed there instead of being hoisted out and kept
// live across the loop, where they would crowd out the accumulators.
template <typename T>
__device__ inline T fresh(T x) {
  asm volatile("" : "+v"(x));
  return x;
}

// The accumulators of the dK/dV and dQ products live in AGPRs for the whole
// loop (mma_acc, attn_ks.hpp): the compiler sees no MFMA there and cannot
// copy them between register files.  Before anything else reads them: the
// wait states an MFMA result needs, then a tie of every register.
template <int N>
__device__ inline void fence_accs(f32x4 (&a)[2][N], f32x4 (&b)[2][N]) {
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < N; ++j) {
      asm volatile("" : "+a"(a[i][j]));
      asm volatile("" : "+a"(b[i][j]));
    }
}
template <int N>
__device__ inline void fence_accs(f32x4 (&a)[2][N]) {
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < N; ++j) asm volatile("" : "+a"(a[i][j]));
}

// ds_write_b128 of N accumulators (AGPRs) at addr + 1024 db.
template <int N, int... DB>
__device__ inline void write_acc_row(unsigned addr, const f32x4 (&acc)[N],
                                     std::integer_sequence<int, DB...>) {
  (write_acc<1024 * DB>(addr, acc[DB]), ...);
}

// 16 bytes from global memory, issued from inline assembly: the compiler
// neither waits for it nor counts it; the caller waits with vm_wait<N>, N
// counting the vector-memory instructions issued after it (LDS DMA ones
// included, which the compiler's own wait counting leaves out).
__device__ inline f32x4 gload16(const void* p) {
  f32x4 r;
  asm volatile("global_load_dwordx4 %0, %1, off" : "=v"(r) : "v"(p) : "memory");
  return r;
}
template <int N>
__device__ inline void vm_wait() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0)" ::"i"(N) : "memory");
}

// Zero in AGPRs, and a tie of every accumulator to an AGPR at the top of
// each loop iteration: the loop-carried values then have AGPRs as their
// home (otherwise the compiler may carry them in VGPRs across the back edge
// and copy all of them between the files every iteration).
template <int N>
__device__ inline void zero_accs(f32x4 (&a)[2][N]) {
  const f32x4 z = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < N; ++j) asm volatile("" : "=a"(a[i][j]) : "0"(z));
}
template <int N>
__device__ inline void home_accs(f32x4 (&a)[2][N]) {
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < N; ++j) asm volatile("" : "+a"(a[i][j]));
}

// Per-lane byte offsets inside a swizzled [rows][D] bf16 tile.
//   frag: row c, piece 4 kk + g (the A or B operand of a 16x16x32 MFMA);
//     rows 16 .. 31 of a block at + 16 * 2D (same swizzle).
//   tr:   ds_read_b64_tr_b16 of column block db: lane (g, c) addresses row
//     4 g + c / 4, columns 16 db + 4 (c % 4) .. + 3, and receives rows
//     4 g .. 4 g + 3 of column 16 db + c; rows 16 .. 31 at + 16 * 2D.
// Both swizzles are XORs of the piece index, so the offsets for k-step kk
// and column block db follow from those of 0 by an XOR with 64 kk and 32 db
// (frag_off(c, g, kk) = frag_off(c, g, 0) ^ 64 kk, tr_off likewise ^ 32 db).
template <int D>
__device__ inline unsigned frag_off(int c, int g, int kk) {
  return static_cast<unsigned>(c * 2 * D + 16 * ((4 * kk + g) ^ swz<D>(c)));
}
template <int D>
__device__ inline unsigned tr_off(int c, int g, int db) {
  const int row = 4 * g + (c >> 2);
  return static_cast<unsigned>(row * 2 * D + 16 * ((2 * db + ((c & 3) >> 1)) ^ swz<D>(row)) +
                               8 * (c & 1));
}

// 32 rows of a [T][H][D] bf16 tensor (row stride rowb bytes) into a
// swizzled [32][D] LDS tile by DMA (buffer_load ... lds, 16 bytes per lane):
// instruction n fills bytes 1024 n .. of dst, lane l piece l % (D/8) of row
// n (64 / (D/8)) + l / (D/8), from global piece slot ^ swz(row).  Rows past
// nvalid lie outside the buffer's range and arrive as zeros.  The per-lane
// offsets are computed here, at the call (a few VALU operations), not held
// in registers across a loop.  Completion is tracked by vmcnt only.
template <int D>
__device__ inline void dma32(const bf16* src, int rowb, int nvalid, unsigned char* dst, int lane) {
#if defined(__HIP_DEVICE_COMPILE__)
  using L = DmaShape<D>;
  const unsigned long long a = reinterpret_cast<unsigned long long>(src);
  const unsigned long long au =
      (static_cast<unsigned long long>(__builtin_amdgcn_readfirstlane(static_cast<int>(a >> 32))) << 32) |
      static_cast<unsigned>(__builtin_amdgcn_readfirstlane(static_cast<int>(a & 0xffffffffu)));
  const int nv = __builtin_amdgcn_readfirstlane(nvalid < 0 ? 0 : nvalid < kChunk ? nvalid : kChunk);
  const __amdgpu_buffer_rsrc_t rs =
      __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void*>(au), (short)0, nv * rowb, kBufferWord3);
  const int ln = fresh(lane);
  const int rl = ln / L::PPR, slot = ln % L::PPR;
#pragma unroll
  for (int n = 0; n < L::NI; ++n) {
    const int r = n * L::RPI + rl;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (GLACIER_LDS void*)(dst + 1024 * n), 16,
                                             r * rowb + 16 * (slot ^ swz<D>(r)), 0, 0, 0);
  }
#endif
}

// bf16x8 from two 4-element halves.
__device__ inline bf16x8 join(bf16x4 lo, bf16x4 hi) {
  bf16x8 r;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    r[i] = lo[i];
    r[4 + i] = hi[i];
  }
  return r;
}

// ---------------------------------------------------------------------------
// bwd_stats: grid (tokens / rows per workgroup, query heads), one 16-lane
// (D=128) or 8-lane (D=64) group per (token, head) row; each lane multiplies
// 8 elements of dO and O in order, the group adds the partials in a fixed
// order.  The row's lse is loaded with its dO and O (no division by a
// runtime value before any load).
// ---------------------------------------------------------------------------
template <int D>
__global__ __launch_bounds__(256) void bwd_stats_kernel(const bf16* __restrict__ d_out,
                                                        const bf16* __restrict__ out,
                                                        const float* __restrict__ lse,
                                                        float2* __restrict__ stats,
                                                        int total_tokens, int n_heads_q) {
  constexpr int LPR = D / 8;      // lanes per row
  constexpr int RPW = 256 / LPR;  // rows (tokens) per workgroup
  const int tok = blockIdx.x * RPW + threadIdx.x / LPR;
  const int h = blockIdx.y;
  const int part = threadIdx.x % LPR;
  const int tt = tok < total_tokens ? tok : total_tokens - 1;  // every lane of a row group stays active
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
// dK/dV tile
// ---------------------------------------------------------------------------
template <int D>
__device__ inline void b2_dkdv(const TileDesc td, const bf16* __restrict__ q_rot,
                               const bf16* __restrict__ d_out, const bf16* __restrict__ k_rot,
                               const bf16* __restrict__ v, const float2* __restrict__ stats,
                               bf16* __restrict__ wk, bf16* __restrict__ wv, int total_tokens,
                               int n_heads_q, int n_heads_kv, int h, int kvh, float scale_log2,
                               float scale, unsigned char* smem) {
  using Lay = B2Layout<D>;
  constexpr int NKD = D / 32, NDB = D / 16;
  const int w = wave_id(), lane = threadIdx.x & 63;
  GL_STAMP(kKernBwd, 0);
  GL_STAMP_VALUE(kKernBwd, 31, td.tile);
  const int kh = w & 1, qg = w >> 1;
  const int k0 = kTile * td.tile;                          // the tile's first key
  const int kw = k0 + 32 * kh;                             // this wave's first key
  const int nst = (td.len - k0 + kChunk - 1) / kChunk;     // 32-query stages from k0 on
  const int nit = (nst + kGroups - 1) / kGroups;
  const long qstride = (long)n_heads_q * D, kvstride = (long)n_heads_kv * D;
  const int qrowb = static_cast<int>(qstride * 2), kvrowb = static_cast<int>(kvstride * 2);
  const bf16* qb0 = q_rot + ((long)td.tok0 * n_heads_q + h) * D;
  const bf16* ob0 = d_out + ((long)td.tok0 * n_heads_q + h) * D;
  const float2* sb0 = stats + (long)h * total_tokens + td.tok0;
  const unsigned sbase = static_cast<unsigned>(reinterpret_cast<uintptr_t>((GLACIER_LDS void*)smem));
  auto slot_at = [&](int it) {
    return Lay::KTILE + Lay::VTILE + (2 * qg + (it & 1)) * Lay::SLOT_KV;
  };
  // stage n (queries k0 + 32 n ..) into this group's slot for iteration it:
  // the key-half-0 wave copies Q, the other dO
  auto issue = [&](int n, int it) {
    const int q0 = k0 + kChunk * n;
    unsigned char* dst = smem + slot_at(it);
    if (kh == 0)
      dma32<D>(qb0 + (long)q0 * qstride, qrowb, td.len - q0, dst, lane);
    else
      dma32<D>(ob0 + (long)q0 * qstride, qrowb, td.len - q0, dst + Lay::CB, lane);
  };

  // Prologue: the tile's K rows (waves 0 and 1, one chunk each) and V rows
  // (waves 2 and 3), each group's first stage.
  if (w < 4) {
    const int half = w & 1, r0 = k0 + kChunk * half;
    const bf16* src = (w < 2 ? k_rot : v) + ((long)(td.tok0 + r0) * n_heads_kv + kvh) * D;
    dma32<D>(src, kvrowb, td.len - r0, smem + (w < 2 ? 0 : Lay::KTILE) + Lay::CB * half, lane);
  }
  if (qg < nst) issue(qg, 0);
  f32x4 acc_dk[2][NDB], acc_dv[2][NDB];
  zero_accs(acc_dk);
  zero_accs(acc_dv);
  const unsigned kaddr = sbase + 32 * kh * 2 * D;  // this wave's 32 K rows
  const unsigned vaddr = kaddr + Lay::KTILE;       // and V rows
  wait_vmem_all();
  __syncthreads();
  GL_STAMP(kKernBwd, 1);

  // One stage: queries q0 .. q0 + 31 against this wave's keys kw .. kw + 31.
  // k-step outer: each K and V fragment is read once per stage and feeds
  // both 16-query blocks; the reads of step kk + 1 are issued before the
  // MFMAs of step kk (one step of LDS latency hidden).  mask: the diagonal
  // stage, or one that runs past the sequence end; masked elements get
  // P = dS = 0 by selection, so no value of a masked row (its row stats are
  // those of another row, or padding) reaches a sum.
  auto stage = [&](int q0, unsigned slot, bool mask, const f32x4 (&st2)[2][2]) {
    // every lane-dependent value is derived from the lane id here, so that
    // only the lane id itself stays live across the loop
    const int ln = fresh(lane), cq = ln & 15, gq = ln >> 4;
    const unsigned fo0 = frag_off<D>(cq, gq, 0), to0 = tr_off<D>(cq, gq, 0);
    const unsigned qa = sbase + slot, oa = qa + Lay::CB;
    f32x4 s[2][2], dp[2][2];  // [query block][key block]
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
      for (int b = 0; b < 2; ++b) s[a][b] = dp[a][b] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    // fragments of one k-step: K, V (two key blocks), Q, dO (two query blocks)
    struct Frags {
      bf16x8 k[2], v[2], q[2], o[2];
    };
    auto issue_frags = [&](Frags& f, unsigned fo) {
      f.k[0] = read_b128_async<0>(kaddr + fo);
      f.k[1] = read_b128_async<32 * D>(kaddr + fo);
      f.q[0] = read_b128_async<0>(qa + fo);
      f.q[1] = read_b128_async<32 * D>(qa + fo);
      f.v[0] = read_b128_async<0>(vaddr + fo);
      f.v[1] = read_b128_async<32 * D>(vaddr + fo);
      f.o[0] = read_b128_async<0>(oa + fo);
      f.o[1] = read_b128_async<32 * D>(oa + fo);
    };
    auto tie_frags = [&](Frags& f) {
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        tie(f.k[i]); tie(f.v[i]); tie(f.q[i]); tie(f.o[i]);
      }
    };
    Frags cur, nxt;
    issue_frags(cur, fo0);
#pragma unroll
    for (int kk = 0; kk < NKD; ++kk) {
      if (kk + 1 < NKD) {
        issue_frags(nxt, fo0 ^ (64u * (kk + 1)));
        lgkm_wait<8>();  // this step's 8 reads; the next step's stay in flight
      } else {
        lgkm_wait0();
      }
      tie_frags(cur);
#pragma unroll
      for (int qb = 0; qb < 2; ++qb)
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
          s[qb][kb] = Mfma<bf16>::mma(cur.q[qb], cur.k[kb], s[qb][kb]);
          dp[qb][kb] = Mfma<bf16>::mma(cur.o[qb], cur.v[kb], dp[qb][kb]);
        }
      if (kk + 1 < NKD) cur = nxt;
    }
    __builtin_amdgcn_sched_barrier(0);
    // dV^T += dO^T P and dK^T += Q^T dS (below): each transposed A fragment
    // feeds both key blocks.  The reads of column blocks 0 .. TRD - 2 are
    // issued here, so the exponentials hide their latency; in the loop,
    // TRD - 1 blocks' reads stay in flight during each block's MFMAs.
    constexpr int TRD = 3;
    bf16x4 t[TRD][4];
    auto issue_tr = [&](bf16x4 (&x)[4], unsigned to) {
      x[0] = read_tr_async<0>(oa + to);
      x[1] = read_tr_async<32 * D>(oa + to);
      x[2] = read_tr_async<0>(qa + to);
      x[3] = read_tr_async<32 * D>(qa + to);
    };
#pragma unroll
    for (int db = 0; db + 1 < TRD; ++db) issue_tr(t[db], to0 ^ (32u * db));
    __builtin_amdgcn_sched_barrier(0);
    float pv[2][2][4], dsv[2][2][4];  // [query block][key block][row]
#pragma unroll
    for (int qb = 0; qb < 2; ++qb)
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          // (nlse2, D) of query 4 g + r: elements 2 (r % 2), 2 (r % 2) + 1 of
          // the block's stats vector r / 2
          const float nl = st2[qb][r >> 1][2 * (r & 1)], dr = st2[qb][r >> 1][2 * (r & 1) + 1];
          pv[qb][kb][r] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[qb][kb][r], scale_log2, nl));
          dsv[qb][kb][r] = pv[qb][kb][r] * (dp[qb][kb][r] - dr);
        }
    // the mask's compares and selects only in the (few) stages that need it:
    // a uniform branch, not a select in every stage
    if (mask) {
#pragma unroll
      for (int qb = 0; qb < 2; ++qb) {
        const int qi0 = q0 + 16 * qb + 4 * gq;  // the lane's first query of the block
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int r = 0; r < 4; ++r)
            if (!(kw + 16 * kb + cq <= qi0 + r && qi0 + r < td.len))
              pv[qb][kb][r] = dsv[qb][kb][r] = 0.0f;
      }
    }
    bf16x8 pB[2], dsB[2];
#pragma unroll
    for (int qb = 0; qb < 2; ++qb)
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          pB[kb][4 * qb + r] = (bf16)pv[qb][kb][r];
          dsB[kb][4 * qb + r] = (bf16)dsv[qb][kb][r];
        }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
      bf16x4 (&x)[4] = t[db % TRD];
      const int ahead = db + TRD - 1;  // the block whose reads go out now
      if (ahead < NDB) issue_tr(t[ahead % TRD], to0 ^ (32u * ahead));
      lgkm_wait_n(4 * ((ahead < NDB ? ahead : NDB - 1) - db));
      tie(x[0]); tie(x[1]); tie(x[2]); tie(x[3]);
      const bf16x8 ao = join(x[0], x[1]), aq = join(x[2], x[3]);
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        mma_acc(acc_dv[kb][db], ao, pB[kb]);
        mma_acc(acc_dk[kb][db], aq, dsB[kb]);
      }
    }
  };

  for (int it = 0; it < nit; ++it) {
    home_accs(acc_dk);
    home_accs(acc_dv);
    const int n = qg + kGroups * it;
    const bool work = n < nst && kw < td.len && n >= kh;
    // row stats (nlse2, D) of queries q0 + 16 qb + 4 g .. + 3 (two 16-byte
    // loads per block), issued before the next stage's DMA and waited for
    // with a count that leaves that DMA in flight (loads complete in order)
    f32x4 st[2][2];
    if (work) {
      const int q0 = k0 + kChunk * n, gq = fresh(lane) >> 4;
#pragma unroll
      for (int qb = 0; qb < 2; ++qb) {
        const float2* sp = sb0 + q0 + 16 * qb + 4 * gq;
        st[qb][0] = gload16(sp);
        st[qb][1] = gload16(sp + 2);
      }
    }
    const bool more = n + kGroups < nst;
    if (more) issue(n + kGroups, it + 1);
    __builtin_amdgcn_sched_barrier(0);
    // stage n against keys kw..: all masked when its last query precedes the
    // first key (n < kh); the diagonal stage (n == kh) and a stage past the
    // sequence end take the mask
    if (work) {
      if (more)
        vm_wait<DmaShape<D>::NI>();  // every load but the DMA just issued
      else
        vm_wait<0>();
#pragma unroll
      for (int qb = 0; qb < 2; ++qb) {
        tie(st[qb][0]);
        tie(st[qb][1]);
      }
      const int q0 = k0 + kChunk * n;
      stage(q0, slot_at(it), n == kh || q0 + kChunk > td.len, st);
    }
    if (it < 16) GL_STAMP(kKernBwd, 4 + it);
    wait_vmem_all();
    __syncthreads();
  }
  GL_STAMP(kKernBwd, 20);

  fence_accs(acc_dk, acc_dv);
  // Merge: every wave writes its sums straight from the AGPRs into region
  // (group, key half) of LDS; then all threads add the four groups of each
  // element in group order and store this head's partial as whole rows
  // (dK first, then dV).
  constexpr int NF4 = 2 * NDB;                 // f32x4 accumulators per tensor per lane
  constexpr int REG = NF4 * 64 * 16;           // bytes of one wave's region
  const unsigned mine = sbase + static_cast<unsigned>((qg * 2 + kh) * REG + lane * 16);
  auto merge_store = [&](f32x4 (&acc)[2][NDB], bf16* dst, float mul) {
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      write_acc_row<NDB>(mine + kb * NDB * 1024, acc[kb], std::make_integer_sequence<int, NDB>{});
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __syncthreads();
    // Each thread takes whole region slots (f32x4 j4 of source lane sl, in
    // both key halves' regions), so a wave reads 64 consecutive 16-byte
    // slots: no LDS bank conflicts.  Slot (j4 = kb NDB + db, sl = 16 g + c)
    // holds elements 16 db + 4 g .. + 3 of key 16 kb + c of the key half.
    for (int i = threadIdx.x; i < 2 * NF4 * 64; i += kB2Threads) {
      const int khr = i / (NF4 * 64), j = i % (NF4 * 64);  // key half, slot in its region
      const int j4 = j >> 6, sl = j & 63;
      const int kbr = j4 / NDB, db = j4 % NDB, gg = sl >> 4, cr = sl & 15;
      const unsigned off = static_cast<unsigned>(j * 16);
      f32x4 x = lds_f4<0>(sbase + static_cast<unsigned>(khr * REG) + off);
      f32x4 y1 = lds_f4<0>(sbase + static_cast<unsigned>((2 + khr) * REG) + off);
      f32x4 y2 = lds_f4<0>(sbase + static_cast<unsigned>((4 + khr) * REG) + off);
      f32x4 y3 = lds_f4<0>(sbase + static_cast<unsigned>((6 + khr) * REG) + off);
      lgkm_wait0();
      tie(x); tie(y1); tie(y2); tie(y3);
      x += y1;
      x += y2;
      x += y3;
      const int key = k0 + 32 * khr + 16 * kbr + cr;
      if (key < td.len)
        store4(dst + ((long)(td.tok0 + key) * n_heads_q + h) * D + 16 * db + 4 * gg, x * mul);
    }
    __syncthreads();
  };
  merge_store(acc_dk, wk, scale);
  GL_STAMP(kKernBwd, 21);
  merge_store(acc_dv, wv, 1.0f);
  GL_STAMP(kKernBwd, 22);
}

// ---------------------------------------------------------------------------
// dQ tile
// ---------------------------------------------------------------------------
template <int D>
__device__ inline void b2_dq(const TileDesc td, const bf16* __restrict__ q_rot,
                             const bf16* __restrict__ d_out, const bf16* __restrict__ k_rot,
                             const bf16* __restrict__ v, const float2* __restrict__ stats,
                             bf16* __restrict__ dq, const int32_t* __restrict__ pos_of,
                             int total_tokens, int n_heads_q, int n_heads_kv, int h, int kvh,
                             float scale_log2, float scale, const float* __restrict__ cos_t,
                             const float* __restrict__ sin_t, unsigned char* smem) {
  using Lay = B2Layout<D>;
  constexpr int NKD = D / 32, NDB = D / 16, H = D / 2;
  const int w = wave_id(), lane = threadIdx.x & 63;
  GL_STAMP(kKernBwd, 0);
  GL_STAMP_VALUE(kKernBwd, 31, 100 + td.tile);
  const int g = lane >> 4, c = lane & 15;
  const int qh = w & 1, kg = w >> 1;
  const int q0t = kTile * td.tile;                  // the tile's first query
  const int qw = q0t + 32 * qh;                     // this wave's first query
  const int kend = min(td.len, q0t + kTile);        // keys before this (the causal range)
  const int nks = (kend + kChunk - 1) / kChunk;     // 32-key stages
  const int nit = (nks + kGroups - 1) / kGroups;
  const int last_m = (qw) / kChunk;                 // this wave's diagonal stage
  const long qstride = (long)n_heads_q * D, kvstride = (long)n_heads_kv * D;
  const bf16* kb0 = k_rot + ((long)td.tok0 * n_heads_kv + kvh) * D;
  const bf16* vb0 = v + ((long)td.tok0 * n_heads_kv + kvh) * D;
  const unsigned sbase = static_cast<unsigned>(reinterpret_cast<uintptr_t>((GLACIER_LDS void*)smem));
  auto slot_at = [&](int it) { return (2 * kg + (it & 1)) * Lay::SLOT_Q; };
  const int kvrowb = static_cast<int>(kvstride * 2);
  auto issue = [&](int m, int it) {
    const int r0 = kChunk * m;
    unsigned char* dst = smem + slot_at(it);
    if (qh == 0)
      dma32<D>(kb0 + (long)r0 * kvstride, kvrowb, td.len - r0, dst, lane);
    else
      dma32<D>(vb0 + (long)r0 * kvstride, kvrowb, td.len - r0, dst + Lay::CB, lane);
  };
  if (kg < nks) issue(kg, 0);
  // The tile's 64 Q rows and 64 dO rows, once per workgroup by DMA, into the
  // second slots of groups 0 and 1 (first written by the loop's first
  // prefetch, after the barrier below): the key-group-0 waves copy Q, the
  // key-group-1 waves dO, one 32-row half each.
  const unsigned qslot = Lay::SLOT_Q, oslot = 3 * Lay::SLOT_Q;
  if (kg < 2) {
    const int r0 = q0t + 32 * qh;
    const bf16* src = (kg == 0 ? q_rot : d_out) + ((long)(td.tok0 + r0) * n_heads_q + h) * D;
    dma32<D>(src, static_cast<int>(qstride * 2), td.len - r0,
             smem + (kg == 0 ? qslot : oslot) + Lay::CB * qh, lane);
  }
  // this wave's queries' row stats (clamped to the sequence: rows past its
  // end are computed but never stored)
  float nl[2], dr[2];
#pragma unroll
  for (int qb = 0; qb < 2; ++qb) {
    const int qi = min(qw + 16 * qb + c, td.len - 1);
    const float2 st = stats[(long)h * total_tokens + td.tok0 + qi];
    nl[qb] = st.x;
    dr[qb] = st.y;
  }
  f32x4 acc[2][NDB];
  zero_accs(acc);
  wait_vmem_all();
  __syncthreads();
  // This wave's Q and dO fragments (B operands: lane (g, c) holds elements
  // 32 kk + 8 g .. of query qw + 16 qb + c), from the staged rows.
  bf16x8 qf[2][NKD], df[2][NKD];
  {
    const unsigned fo0 = frag_off<D>(c, g, 0);
    const unsigned qa = sbase + qslot + 32 * qh * 2 * D, oa = sbase + oslot + 32 * qh * 2 * D;
#pragma unroll
    for (int kk = 0; kk < NKD; ++kk) {
      const unsigned fo = fo0 ^ (64u * kk);
      qf[0][kk] = read_b128_async<0>(qa + fo);
      qf[1][kk] = read_b128_async<32 * D>(qa + fo);
      df[0][kk] = read_b128_async<0>(oa + fo);
      df[1][kk] = read_b128_async<32 * D>(oa + fo);
    }
    lgkm_wait0();
#pragma unroll
    for (int qb = 0; qb < 2; ++qb)
#pragma unroll
      for (int kk = 0; kk < NKD; ++kk) {
        tie(qf[qb][kk]);
        tie(df[qb][kk]);
      }
  }
  wait_vmem_all();
  __syncthreads();
  GL_STAMP(kKernBwd, 1);

  // One stage: keys 32 m .. + 31 against this wave's queries; mask: the
  // diagonal stage.
  auto stage = [&](int m, unsigned slot, bool mask) {
    const int ln = fresh(lane), cq = ln & 15, gq = ln >> 4;
    const unsigned fo0 = frag_off<D>(cq, gq, 0), to0 = tr_off<D>(cq, gq, 0);
    const unsigned ka = sbase + slot, va = ka + Lay::CB;
    f32x4 s[2][2], dp[2][2];  // [key block][query block]
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
      for (int b = 0; b < 2; ++b) s[a][b] = dp[a][b] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    // K and V fragments of one k-step (two key blocks each), read one step
    // ahead of their MFMAs
    bf16x8 fr[2][4];
    auto issue_frags = [&](bf16x8 (&f)[4], unsigned fo) {
      f[0] = read_b128_async<0>(ka + fo);
      f[1] = read_b128_async<32 * D>(ka + fo);
      f[2] = read_b128_async<0>(va + fo);
      f[3] = read_b128_async<32 * D>(va + fo);
    };
    issue_frags(fr[0], fo0);
#pragma unroll
    for (int kk = 0; kk < NKD; ++kk) {
      bf16x8 (&f)[4] = fr[kk & 1];
      if (kk + 1 < NKD) {
        issue_frags(fr[(kk + 1) & 1], fo0 ^ (64u * (kk + 1)));
        lgkm_wait<4>();
      } else {
        lgkm_wait0();
      }
      tie(f[0]); tie(f[1]); tie(f[2]); tie(f[3]);
#pragma unroll
      for (int qb = 0; qb < 2; ++qb) {
        s[0][qb] = Mfma<bf16>::mma(f[0], qf[qb][kk], s[0][qb]);
        s[1][qb] = Mfma<bf16>::mma(f[1], qf[qb][kk], s[1][qb]);
        dp[0][qb] = Mfma<bf16>::mma(f[2], df[qb][kk], dp[0][qb]);
        dp[1][qb] = Mfma<bf16>::mma(f[3], df[qb][kk], dp[1][qb]);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    // dQ^T += K^T dS^T (below): each transposed K fragment feeds both query
    // blocks.  The reads of column blocks 0 .. TRD - 2 are issued here, so
    // the exponentials hide their latency; in the loop, TRD - 1 blocks'
    // reads stay in flight during each block's MFMAs.
    constexpr int TRD = 3;
    bf16x4 t[TRD][2];
#pragma unroll
    for (int db = 0; db + 1 < TRD; ++db) {
      t[db][0] = read_tr_async<0>(ka + (to0 ^ (32u * db)));
      t[db][1] = read_tr_async<32 * D>(ka + (to0 ^ (32u * db)));
    }
    __builtin_amdgcn_sched_barrier(0);
    float pv[2][2][4];  // [key block][query block][row]
#pragma unroll
    for (int qb = 0; qb < 2; ++qb)
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          pv[kb][qb][r] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[kb][qb][r], scale_log2, nl[qb]));
    if (mask) {  // a uniform branch: the compares only in the diagonal stage
#pragma unroll
      for (int qb = 0; qb < 2; ++qb)
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int r = 0; r < 4; ++r)
            if (kChunk * m + 16 * kb + 4 * gq + r > qw + 16 * qb + cq) pv[kb][qb][r] = 0.0f;
    }
    bf16x8 dsB[2];
#pragma unroll
    for (int qb = 0; qb < 2; ++qb)
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          dsB[qb][4 * kb + r] = (bf16)(pv[kb][qb][r] * (dp[kb][qb][r] - dr[qb]));
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
      bf16x4 (&x)[2] = t[db % TRD];
      const int ahead = db + TRD - 1;
      if (ahead < NDB) {
        const unsigned to = to0 ^ (32u * ahead);
        t[ahead % TRD][0] = read_tr_async<0>(ka + to);
        t[ahead % TRD][1] = read_tr_async<32 * D>(ka + to);
      }
      lgkm_wait_n(2 * ((ahead < NDB ? ahead : NDB - 1) - db));
      tie(x[0]); tie(x[1]);
      const bf16x8 a = join(x[0], x[1]);
#pragma unroll
      for (int qb = 0; qb < 2; ++qb) mma_acc(acc[qb][db], a, dsB[qb]);
    }
  };

  for (int it = 0; it < nit; ++it) {
    home_accs(acc);
    const int m = kg + kGroups * it;
    if (m + kGroups < nks) issue(m + kGroups, it + 1);
    __builtin_amdgcn_sched_barrier(0);
    if (m < nks && qw < td.len && m <= last_m) stage(m, slot_at(it), m == last_m);
    if (it < 16) GL_STAMP(kKernBwd, 4 + it);
    wait_vmem_all();
    __syncthreads();
  }
  GL_STAMP(kKernBwd, 20);

  fence_accs(acc);
  // Merge: every wave writes its sums from the AGPRs into region (group,
  // query half); then all threads add the four key groups of each element in
  // group order, scale, apply the inverse RoPE at the query's position and
  // store rows of dq.  A thread takes elements d .. d + 3 and d + D/2 ..
  // (the rotation pairs) of one query.
  constexpr int NF4 = 2 * NDB;
  constexpr int REG = NF4 * 64 * 16;
  const unsigned mine = sbase + static_cast<unsigned>((kg * 2 + qh) * REG + lane * 16);
#pragma unroll
  for (int qb = 0; qb < 2; ++qb)
    write_acc_row<NDB>(mine + qb * NDB * 1024, acc[qb], std::make_integer_sequence<int, NDB>{});
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  __syncthreads();
  // Each thread takes region slots (f32x4 j4 = qb NDB + db, db < NDB / 2,
  // of source lane sl) and the slot of column block db + NDB / 2 (the
  // rotation partners d, d + D/2), in the query half's four group regions:
  // a wave reads 64 consecutive 16-byte slots, free of bank conflicts.
  for (int i = threadIdx.x; i < 2 * NDB * 64; i += kB2Threads) {  // 2 halves x 2 qb x NDB/2 x 64
    const int qhr = i / (NDB * 64), j = i % (NDB * 64);
    const int jh = j >> 6, sl = j & 63;                  // jh = qb (NDB/2) + db
    const int qbr = jh / (NDB / 2), db = jh % (NDB / 2), gg = sl >> 4, cr = sl & 15;
    const unsigned off0 = static_cast<unsigned>(((qbr * NDB + db) * 64 + sl) * 16);
    const unsigned off1 = off0 + (NDB / 2) * 64 * 16;   // column block db + NDB / 2
    f32x4 lo[4], hi[4];
#pragma unroll
    for (int u = 0; u < kGroups; ++u) {
      lo[u] = lds_f4<0>(sbase + static_cast<unsigned>((2 * u + qhr) * REG) + off0);
      hi[u] = lds_f4<0>(sbase + static_cast<unsigned>((2 * u + qhr) * REG) + off1);
    }
    lgkm_wait0();
#pragma unroll
    for (int u = 0; u < kGroups; ++u) {
      tie(lo[u]);
      tie(hi[u]);
    }
#pragma unroll
    for (int u = 1; u < kGroups; ++u) {
      lo[0] += lo[u];
      hi[0] += hi[u];
    }
    const int qi = q0t + 32 * qhr + 16 * qbr + cr;
    const int d0 = 16 * db + 4 * gg;  // elements d0 .. d0 + 3 and H + d0 ..
    if (qi < td.len) {
      const long pos = pos_of != nullptr ? pos_of[td.tok0 + qi] : qi;
      const f32x4 cs = *reinterpret_cast<const f32x4*>(cos_t + pos * H + d0);
      const f32x4 sn = *reinterpret_cast<const f32x4*>(sin_t + pos * H + d0);
      const f32x4 a = lo[0] * scale, b = hi[0] * scale;
      f32x4 y0, y1;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        float u0, u1;
        rope_inv(a[r], b[r], cs[r], sn[r], u0, u1);
        y0[r] = u0;
        y1[r] = u1;
      }
      bf16* row_p = dq + ((long)(td.tok0 + qi) * n_heads_q + h) * D;
      store4(row_p + d0, y0);
      store4(row_p + H + d0, y1);
    }
  }
  GL_STAMP(kKernBwd, 22);
}

// grid (Hq/Hkv, Hkv, 2 n_tiles); z indexes the tile table (both kinds,
// longest expected first).
template <int D>
__global__ __launch_bounds__(kB2Threads) void attn_bwd2_kernel(
    const bf16* __restrict__ q_rot, const bf16* __restrict__ d_out, const bf16* __restrict__ k_rot,
    const bf16* __restrict__ v, const float2* __restrict__ stats, bf16* __restrict__ dq,
    bf16* __restrict__ wk, bf16* __restrict__ wv, const TileDesc* __restrict__ tiles_bwd,
    const int32_t* __restrict__ pos_of, int total_tokens, float scale_log2, float scale,
    const float* __restrict__ cos_t, const float* __restrict__ sin_t) {
  extern __shared__ __align__(16) unsigned char smem_raw[];
  const int ratio = gridDim.x, n_heads_kv = gridDim.y, n_heads_q = ratio * n_heads_kv;
  const int kvh = blockIdx.y, h = kvh * ratio + blockIdx.x;
  const TileDesc td = tiles_bwd[blockIdx.z];
  if (td.kind == kTileDkDv)
    b2_dkdv<D>(td, q_rot, d_out, k_rot, v, stats, wk, wv, total_tokens, n_heads_q, n_heads_kv, h,
               kvh, scale_log2, scale, smem_raw);
  else
    b2_dq<D>(td, q_rot, d_out, k_rot, v, stats, dq, pos_of, total_tokens, n_heads_q, n_heads_kv, h,
             kvh, scale_log2, scale, cos_t, sin_t, smem_raw);
}

}  // namespace

template <int D>
hipError_t launch_bwd2(const BwdLaunch& a, hipStream_t st, KernelTimer* tm) {
  const int ratio = a.n_heads_q / a.n_heads_kv;
  float2* stats = static_cast<float2*>(a.stats);
  {
    constexpr int rows_per_wg = 256 / (D / 8);
    const dim3 grid(static_cast<unsigned>((a.total_tokens + rows_per_wg - 1) / rows_per_wg),
                    a.n_heads_q);
    LaunchTiming t(tm, kKernBwdStats);
    GL_LAUNCH(t, (bwd_stats_kernel<D>), grid, dim3(256), 0, st,
              static_cast<const bf16*>(a.d_out), static_cast<const bf16*>(a.out), a.lse, stats,
              a.total_tokens, a.n_heads_q);
    GL_CHECK(hipGetLastError());
    t.launched();
  }
  {
    auto fn = attn_bwd2_kernel<D>;
    constexpr size_t lds = B2Layout<D>::BYTES;
    GL_CHECK(allow_lds(fn, lds));
    LaunchTiming t(tm, kKernBwd);
    GL_LAUNCH(t, fn, dim3(ratio, a.n_heads_kv, 2 * a.n_tiles), dim3(kB2Threads), lds, st,
              static_cast<const bf16*>(a.q_rot), static_cast<const bf16*>(a.d_out),
              static_cast<const bf16*>(a.k_rot), static_cast<const bf16*>(a.v),
              static_cast<const float2*>(stats), static_cast<bf16*>(a.dq),
              static_cast<bf16*>(a.wk), static_cast<bf16*>(a.wv), a.tiles_bwd,
              a.single_seq ? nullptr : a.pos_of, a.total_tokens, a.scale_log2, a.scale, a.cos_t,
              a.sin_t);
    GL_CHECK(hipGetLastError());
    t.launched();
  }
  return hipSuccess;
}

template hipError_t launch_bwd2<64>(const BwdLaunch&, hipStream_t, KernelTimer*);
template hipError_t launch_bwd2<128>(const BwdLaunch&, hipStream_t, KernelTimer*);

}  // namespace glacier

#ifdef GLACIER_PHASE_STAMPS
// Profiling builds only: copies this file's phase stamps (the bf16
// backward's) to host memory.
extern "C" int glacier_attn_debug_stamps_bwd(void* host, size_t bytes) {
  return static_cast<int>(hipMemcpyFromSymbol(host, HIP_SYMBOL(glacier::glacier_stamps), bytes));
}
#endif
