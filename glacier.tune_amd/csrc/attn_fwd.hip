// attn_fwd.hip -- the bf16-MFMA attention forward (gfx950, wave64).
//
// GpuLoraEngine.Forward.cs:401-465 (tune_attn_causal_gqa_fwd): for each
// query head and query i, O_i = softmax_j<=i(q_i . k_j / sqrt(D)) V_j and the
// row log-sum-exp, with q rotated here (q_rot written when saving) and K
// already rotated by rope_k.
//
// Key-split waves.  One workgroup of 4 waves (one per SIMD) per (query head,
// 64-query tile).  Every wave holds the whole tile's Q^T fragments (VGPRs)
// and O^T accumulators (AGPRs) and walks its own 32-key chunks of the causal
// range (chunks w, w + 4, w + 8, ...): a K fragment read from LDS feeds four
// MFMAs (one per 16-query block) and so does a V fragment, a quarter of the
// LDS traffic per MFMA of waves that own 16 queries each.
//   * K and V chunks go from L2 straight into the wave's own two-slot LDS
//     rings (buffer_load ... lds, 16 bytes per lane, XOR-swizzled rows), two
//     chunks ahead, with no workgroup barrier inside the loop.
//   * Software pipeline: an iteration issues chunk i + 1's scores while it
//     takes chunk i's exponentials, and chunk i's PV products while it takes
//     chunk i + 1's maxima; the row sums are four more MFMAs against ones.
//   * No rescaling inside the loop: the probabilities are taken against each
//     column's maximum in the wave's first chunk; a later chunk exceeding it
//     by more than 2^16 makes the wave run its chunks again with the true
//     maxima (exact either way; rare).
//   * The four partial states (max, sum, O) are merged per 16-query block by
//     the wave that owns the block, in wave order.
// The compiler's own MFMAs write VGPRs (-mllvm -amdgpu-mfma-vgpr-form,
// build.py); the accumulators are pinned to AGPRs by inline assembly, and
// the LDS reads whose completion the compiler would otherwise tie to the
// DMA are issued from inline assembly with explicit waits.
#include "attn_common.hpp"
#include "attn_ks.hpp"
#include "attn_launch.hpp"

#include <hip/hip_ext.h>

#include <type_traits>
#include <utility>

namespace glacier {
namespace {

constexpr int kFwdWaves = 4;
constexpr float kRescale = 16.0f;  // reference maxima may lag the true ones by 2^16

template <int D>
struct FwdLayout {
  static constexpr int CHUNK = kChunk * D;  // elements of one K or V chunk
  static constexpr int WAVE = 4 * CHUNK;    // a wave's two (K, V) buffers
  static constexpr size_t LOOP = sizeof(bf16) * (kFwdWaves * WAVE + kTile * D);
  static constexpr int OS = D + 4;  // row stride (floats) of the merge area
  static constexpr size_t BYTES = LOOP;  // the merge reuses each wave's ring region
};

template <int N>
__device__ inline void wait_kfrags(bf16x8 (&t)[4][2]) {
  static_assert(N >= 0 && N < 16, "lgkmcnt range");
  asm volatile("s_waitcnt lgkmcnt(%8)"
               : "+v"(t[0][0]), "+v"(t[0][1]), "+v"(t[1][0]), "+v"(t[1][1]), "+v"(t[2][0]),
                 "+v"(t[2][1]), "+v"(t[3][0]), "+v"(t[3][1])
               : "i"(N));
}
template <int N>
__device__ inline void wait_kfrags(bf16x8 (&t)[2][2]) {
  static_assert(N >= 0 && N < 16, "lgkmcnt range");
  asm volatile("s_waitcnt lgkmcnt(%4)" : "+v"(t[0][0]), "+v"(t[0][1]), "+v"(t[1][0]), "+v"(t[1][1]) : "i"(N));
}

// Wait states between the last mma_acc and any other access of the
// accumulators (24 >= the 18 a 16-pass MFMA result needs); every
// accumulator is tied through a volatile asm after the wait, so no access
// moves above it.
template <int NDB, int QB>
__device__ inline void fence_acc(f32x4 (&o)[NDB][QB], f32x4 (&l)[QB]) {
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    asm volatile("" : "+a"(l[qb]));
#pragma unroll
    for (int db = 0; db < NDB; ++db) asm volatile("" : "+a"(o[db][qb]));
  }
}

// the NDB 16-byte pieces of block qb of the accumulators at addr + 64 db
template <int NDB, int QB, int... DB>
__device__ inline void write_acc_block(unsigned addr, const f32x4 (&o)[NDB][QB], int qb,
                                       std::integer_sequence<int, DB...>) {
  (write_acc<64 * DB>(addr, o[DB][qb]), ...);
}

// The arguments the first loads need come first: the 14 dwords up to cos_t
// arrive preloaded in SGPRs (-amdgpu-kernarg-preload-count, build.py), so the
// K/V and Q loads issue without waiting for the kernarg segment.  The sine
// table starts sin_off floats after the cosine table.
template <typename IO, int D, bool VARLEN, int QB>
__global__ __launch_bounds__(kFwdWaves * 64) void attn_fwd_kernel_ks(
    int total_tokens, int n_heads_kv, int group, int sin_off, const bf16* __restrict__ kc,
    const bf16* __restrict__ v, const TileDesc* __restrict__ tiles, const IO* __restrict__ q,
    const float* __restrict__ cos_t, IO* __restrict__ out, float* __restrict__ lse,
    IO* __restrict__ q_rot, float scale_log2) {
  using M = Mfma<bf16>;
  using F = FwdLayout<D>;
  using Frag = M::Frag;
  constexpr int NKD = D / M::KSTEP;
  constexpr int NDB = D / 16;
  constexpr int H = D / 2;
  constexpr int NT = kFwdWaves * 64;
  static_assert(QB == 4 || QB == 2 || QB == 1, "16-query blocks per workgroup");
  constexpr int TR = 16 * QB;       // query rows of the workgroup
  constexpr int NSUB = kTile / TR;  // workgroups per 64-row table entry
  constexpr int NDMA = 2 * (kChunk * D / 512);  // DMA instructions per chunk (K and V)
  static_assert(NDMA < 64, "vmcnt range");
  constexpr unsigned SLOT = F::CHUNK * sizeof(bf16);  // bytes of one ring slot
  extern __shared__ __align__(16) unsigned char smem_raw[];
  bf16* const lds = reinterpret_cast<bf16*>(smem_raw);  // [wave][K ring, V ring], Q

  // grid (group = query heads per KV head, KV heads, tiles): no integer division
  const int n_heads_q = group * n_heads_kv;
  const int kvh = blockIdx.y, h = kvh * group + blockIdx.x;
  const float* const sin_t = cos_t + sin_off;
  // the rows of an entry's later part see more keys and start first
  const int entry = (int)blockIdx.z / NSUB, sub = NSUB - 1 - (int)blockIdx.z % NSUB;
  const TileDesc td =
      VARLEN ? tiles[entry] : TileDesc{0, total_tokens, (total_tokens + kTile - 1) / kTile - 1 - entry, 0};
  const int tid = threadIdx.x, w = wave_id(), lane = tid & 63;
  GL_STAMP(kKernFwd, 0);
  const int g = lane >> 4, c = lane & 15;
  const int q0 = kTile * td.tile + TR * sub;  // the workgroup's first query position
  const int nq = min(TR, td.len - q0);        // its valid queries
  if (nq <= 0) return;  // the part of a short last tile past the sequence's end
  GL_STAMP_VALUE(kKernFwd, 31, q0 / TR);
  const int nch = (q0 + nq + kChunk - 1) / kChunk;  // key chunks of the causal range
  const int nit = __builtin_amdgcn_readfirstlane(nch > w ? (nch - w + kFwdWaves - 1) / kFwdWaves : 0);
  // This wave's LDS: a two-slot ring of K chunks, then one of V chunks
  // (chunk i in slot i & 1).  K of chunk i + 1 is read one iteration ahead of
  // V of chunk i, so the rings refill at different points of an iteration.
  bf16* const kring = lds + w * F::WAVE;
  bf16* const vring = kring + 2 * F::CHUNK;

  // Q: the workgroup's rows are loaded by all threads (coalesced, 8 rotation
  // pairs per thread), rotated in fp32 (rope_fwd) and rounded to bf16,
  // written to LDS (swizzled), from where every wave reads the operand
  // fragments of all TR queries, and later to q_rot as whole rows.  Their
  // loads issue ahead of the K/V DMA: loads return in order, and Q is
  // needed first.
  bf16* const qst = lds + kFwdWaves * F::WAVE;
  constexpr int PPR = H / 8;                // 8-pair pieces per row
  constexpr int QP = TR * PPR;              // pieces of the rows
  constexpr int QI = (QP + NT - 1) / NT;    // pieces per thread
  // Q pieces as loaded (bf16 rows stay packed until the rotation, so that
  // no conversion waits for them before the DMA has issued)
  using QRaw = std::conditional_t<std::is_same_v<IO, bf16>, bf16x8, float[8]>;
  QRaw qx[QI][2];
  float qc[QI][8], qs[QI][8];
  auto load_raw = [](const IO* p, QRaw& x) {
    if constexpr (std::is_same_v<IO, bf16>)
      x = *reinterpret_cast<const bf16x8*>(p);
    else
      load8(p, x);
  };
  const long qrow0 = (long)td.tok0 + q0;
#pragma unroll
  for (int n = 0; n < QI; ++n) {
    const int idx = tid + n * NT;
    if (QP % NT != 0 && idx >= QP) break;
    const int r = idx / PPR, j = idx % PPR;
    const int rr = r < nq ? r : 0;  // rows past the sequence load row 0, rotate zeros
    const long gq = ((qrow0 + rr) * n_heads_q + h) * D + 8 * j;
    load_raw(q + gq, qx[n][0]);
    load_raw(q + gq + H, qx[n][1]);
    const long ti = (long)(q0 + rr) * H + 8 * j;
    load8(cos_t + ti, qc[n]);
    load8(sin_t + ti, qs[n]);
  }

  const long kvstride = (long)n_heads_kv * D;
  const bf16* kbase = kc + ((long)td.tok0 * n_heads_kv + kvh) * D;
  const bf16* vbase = v + ((long)td.tok0 * n_heads_kv + kvh) * D;
  const DmaLanes dl = dma_lanes<D>(kvstride, lane);
  // chunk i of this wave: keys 32 (w + 4 i) .., into ring slot i & 1
  auto dma_k = [&](int i) {
    const int j = w + kFwdWaves * i;
    dma_chunk<D>(dl, kbase + (long)kChunk * j * kvstride, td.len - kChunk * j, kring + (i & 1) * F::CHUNK);
  };
  auto dma_v = [&](int i) {
    const int j = w + kFwdWaves * i;
    dma_chunk<D>(dl, vbase + (long)kChunk * j * kvstride, td.len - kChunk * j, vring + (i & 1) * F::CHUNK);
  };
  if (nit > 0) {
    dma_k(0);
    dma_v(0);
  }
  if (nit > 1) {
    dma_k(1);
    dma_v(1);
  }
  GL_STAMP(kKernFwd, 23);

  float qy[QI][2][8];
#pragma unroll
  for (int n = 0; n < QI; ++n) {
    const int idx = tid + n * NT;
    if (QP % NT != 0 && idx >= QP) break;
    const int r = idx / PPR, j = idx % PPR;
    const bool valid = r < nq;
#pragma unroll
    for (int e = 0; e < 8; ++e)
      rope_fwd(valid ? (float)qx[n][0][e] : 0.0f, valid ? (float)qx[n][1][e] : 0.0f, qc[n][e], qs[n][e],
               qy[n][0][e], qy[n][1][e]);
    const int sw = swz<D>(r);
    store8(qst + r * D + 8 * (j ^ sw), qy[n][0]);
    store8(qst + r * D + 8 * ((PPR + j) ^ sw), qy[n][1]);
  }
  GL_STAMP(kKernFwd, 1);
  __syncthreads();
  Frag qf[QB][NKD];
  {
    const int sq = swz<D>(c);  // rows 16 qb + c
#pragma unroll
    for (int qb = 0; qb < QB; ++qb)
#pragma unroll
      for (int kk = 0; kk < NKD; ++kk)
        qf[qb][kk] = *reinterpret_cast<const bf16x8*>(qst + (16 * qb + c) * D + 8 * ((4 * kk + g) ^ sq));
  }
  GL_STAMP(kKernFwd, 2);

  // Per-lane LDS addresses (bytes, slot 0) of the chunk reads; the slot and
  // the 16-row block go into the instructions' offset fields.  K fragments:
  // row 16 kb + c, piece 4 kk + g.  V transposing reads
  // (ds_read_b64_tr_b16): lane (g, i) addresses row 16 s + 4 g + i / 4,
  // columns 16 db + 4 (i % 4) .. + 3, i.e. piece 2 db + (i % 4) / 2 at
  // element 4 (i % 2) of it.  Row offsets of 16 leave the swizzle unchanged.
  unsigned kaddr[NKD], vaddr[NDB];
  {
    const int sk = swz<D>(c);
    const int vrow = 4 * g + (c >> 2);
    const int sv = swz<D>(vrow);
    const int vpiece = (c & 3) >> 1;
#pragma unroll
    for (int kk = 0; kk < NKD; ++kk) kaddr[kk] = lds_addr(kring + c * D + 8 * ((4 * kk + g) ^ sk));
#pragma unroll
    for (int db = 0; db < NDB; ++db)
      vaddr[db] = lds_addr(vring + vrow * D + 4 * (c & 1) + 8 * ((2 * db + vpiece) ^ sv));
  }

  // O^T accumulators and per-query row sums (MFMA accumulators pinned in
  // AGPRs), the reference maxima the probabilities are taken against.
  f32x4 o[NDB][QB], lsum[QB];
  float m_ref[QB], m_seen[QB];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    // a wave without chunks merges as (kNegBig, 0, 0)
    m_ref[qb] = kNegBig;
    m_seen[qb] = kNegBig;
  }
  bool grew = false;
  bf16x8 ones;
#pragma unroll
  for (int e = 0; e < 8; ++e) ones[e] = (bf16)1.0f;

  // One iteration: chunk i's probabilities, row sums and PV (its scores in
  // sc, its V in slot i & 1), chunk i + 1's scores and maxima (MORE: chunk
  // i + 1 exists; its K is in the other slot), which replace sc.  MASK: chunk
  // i + 1 may reach the diagonal (only a wave's last chunk can).  FETCH:
  // chunk i + 2 exists; its K goes into K(i)'s slot at the start, its V into
  // V(i)'s at the end.  On entry K(i + 1) and V(i) are in LDS or in flight.
  f32x4 sc[2][QB];
  auto iteration = [&](int i, auto more, auto mask, auto fetch) {
    constexpr bool MORE = decltype(more)::value;
    constexpr bool MASK = decltype(mask)::value;
    constexpr bool FETCH = decltype(fetch)::value;
    if constexpr (MORE)
      wait_vmcnt<NDMA / 2>();  // all but V(i + 1)'s DMA
    else
      wait_vmcnt<0>();
    if (i < 6) GL_STAMP(kKernFwd, 4 + 2 * i);
    if constexpr (FETCH) dma_k(i + 2);  // every read of K(i) completed last iteration
    // K fragments of chunk i + 1, then the V^T fragments of chunk i (two
    // transposing reads per 16-row block), all issued before any is used.
    const unsigned vslot = (i & 1) * SLOT, kslot = SLOT - vslot;
    bf16x8 kf[NKD][2];
    if constexpr (MORE) {
#pragma unroll
      for (int kk = 0; kk < NKD; ++kk) {
        kf[kk][0] = read_b128_async<0>(kaddr[kk] + kslot);
        kf[kk][1] = read_b128_async<32 * D>(kaddr[kk] + kslot);
      }
    }
    bf16x4 vt[2 * NDB];
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
      vt[2 * db] = read_tr_async<0>(vaddr[db] + vslot);
      vt[2 * db + 1] = read_tr_async<32 * D>(vaddr[db] + vslot);
    }
    // Part 1: chunk i + 1's score MFMAs with chunk i's probabilities
    // (independent work) interleaved, so that the VALU takes the
    // exponentials while the matrix core runs: one wave per SIMD issues in
    // order, and a run of MFMAs would stall the VALU work behind it.
    f32x4 sn[2][QB];
    if constexpr (MORE) {
      wait_kfrags<(2 * NDB < 15 ? 2 * NDB : 15)>(kf);
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) sn[kb][qb] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    }
    // G groups, each of MPG score MFMAs (m -> kk, kb, qb) and one pair of
    // probabilities (p -> qb, kb, r pair), fenced so the order holds.
    bf16x8 pb[QB];
    constexpr int G = 4 * QB;
    constexpr int MPG = 2 * QB * NKD / G;
    static_assert(MPG * G == 2 * QB * NKD, "score MFMAs per group");
#pragma unroll
    for (int grp = 0; grp < G; ++grp) {
      if constexpr (MORE) {
#pragma unroll
        for (int mm = 0; mm < MPG; ++mm) {
          const int m = grp * MPG + mm;
          const int kk = m / (2 * QB), kb = (m / QB) % 2, qb = m % QB;
          sn[kb][qb] = M::mma(kf[kk][kb], qf[qb][kk], sn[kb][qb]);
        }
      }
      const int qb = grp / 4, kb = (grp / 2) % 2, r0 = 2 * (grp % 2);
#pragma unroll
      for (int r = r0; r < r0 + 2; ++r)
        pb[qb][4 * kb + r] = (bf16)__builtin_amdgcn_exp2f(__builtin_fmaf(sc[kb][qb][r], scale_log2, -m_ref[qb]));
      __builtin_amdgcn_sched_barrier(0);
    }
    wait_tr(vt);
    bf16x8 va[NDB];
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        va[db][r] = vt[2 * db][r];
        va[db][4 + r] = vt[2 * db + 1][r];
      }
    // Part 2: chunk i's row sums and PV products (query block by query
    // block, in pairs behind one wait), with chunk i + 1's maxima in log2
    // units interleaved, EPP score elements after each pair (keys after a
    // query set to -inf first when the chunk may reach the diagonal).
    constexpr int NPAIR = (NDB + 2) / 2;             // pairs of the NDB + 1 products
    constexpr int EPP = (8 + NPAIR - 1) / NPAIR;     // maxima elements per pair
    const int koff = kChunk * (w + kFwdWaves * (i + 1)) - q0;  // chunk i + 1's key 0, from query 0
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      float mloc = -INFINITY;
      // product j: the row sums (j = 0) or O^T block j - 1
      auto acc_of = [&](auto jc) -> f32x4& {
        if constexpr (decltype(jc)::value == 0)
          return lsum[qb];
        else
          return o[decltype(jc)::value - 1][qb];
      };
      auto opa_of = [&](auto jc) -> const bf16x8& {
        if constexpr (decltype(jc)::value == 0)
          return ones;
        else
          return va[decltype(jc)::value - 1];
      };
      static_for<NPAIR>([&](auto pc) {
        constexpr int j0 = 2 * decltype(pc)::value, j1 = j0 + 1;
        using J0 = std::integral_constant<int, j0>;
        using J1 = std::integral_constant<int, (j1 <= NDB ? j1 : j0)>;
        if constexpr (j1 <= NDB)
          mma_acc2(acc_of(J0{}), opa_of(J0{}), pb[qb], acc_of(J1{}), opa_of(J1{}), pb[qb]);
        else
          mma_acc(acc_of(J0{}), opa_of(J0{}), pb[qb]);
        if constexpr (MORE) {
#pragma unroll
          for (int e = EPP * decltype(pc)::value; e < EPP * decltype(pc)::value + EPP && e < 8; ++e) {
            const int kb = e >> 2, r = e & 3;
            if (MASK)
              sn[kb][qb][r] = (koff + 16 * kb + 4 * g + r <= 16 * qb + c) ? sn[kb][qb][r] : -INFINITY;
            mloc = fmaxf(mloc, sn[kb][qb][r]);
          }
          asm volatile("" ::"v"(mloc));  // computed here, not sunk past the products
        }
        __builtin_amdgcn_sched_barrier(0);
      });
      if constexpr (MORE) {
        // lane-local: a chunk exceeds a column's reference iff one of the
        // column's four lanes does, and the maxima seen become the rescue
        // pass's references only after one cross-lane reduction at the end
        const float ml = mloc * scale_log2;
        grew = grew || (ml > m_ref[qb] + kRescale);
        m_seen[qb] = fmaxf(m_seen[qb], ml);
      }
    }
    if constexpr (MORE) {
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) sc[kb][qb] = sn[kb][qb];
    }
    if constexpr (FETCH) {
      __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): every read of V(i) is complete
      __atomic_signal_fence(__ATOMIC_SEQ_CST);
      dma_v(i + 2);
    }
  };

  // Pass 0 takes each column's reference maximum from the wave's first
  // chunk; no rescaling ever happens inside the loop.  If a later chunk's
  // maximum exceeds it by more than 2^16 (rare: probabilities stay finite up
  // to 2^128, and the results are exact either way), the wave runs its
  // chunks again with the maxima it saw as references (pass 1 cannot grow).
#pragma clang loop unroll(disable)
  for (int pass = 0; pass < 2; ++pass) {
    if (pass > 0) {
      __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the last chunk's reads are complete
      __atomic_signal_fence(__ATOMIC_SEQ_CST);
      if (nit > 0) {
        dma_k(0);
        dma_v(0);
      }
      if (nit > 1) {
        dma_k(1);
        dma_v(1);
      }
    }
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      lsum[qb] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int db = 0; db < NDB; ++db) o[db][qb] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    }
    grew = false;
    if (nit > 0) {
      // chunk 0: K(1)'s DMA (issued after K(0), V(0)) may still be in flight
      if (nit > 1)
        wait_vmcnt<NDMA / 2 * 3>();
      else
        wait_vmcnt<NDMA / 2>();
      GL_STAMP(kKernFwd, 18);
      bf16x8 kf[NKD][2];
#pragma unroll
      for (int kk = 0; kk < NKD; ++kk) {
        kf[kk][0] = read_b128_async<0>(kaddr[kk]);
        kf[kk][1] = read_b128_async<32 * D>(kaddr[kk]);
      }
      wait_kfrags<0>(kf);
      GL_STAMP(kKernFwd, 19);
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) sc[kb][qb] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int kk = 0; kk < NKD; ++kk)
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int qb = 0; qb < QB; ++qb) sc[kb][qb] = M::mma(kf[kk][kb], qf[qb][kk], sc[kb][qb]);
      const int koff = kChunk * w - q0;
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) {
        float mloc = -INFINITY;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            sc[kb][qb][r] = (koff + 16 * kb + 4 * g + r <= 16 * qb + c) ? sc[kb][qb][r] : -INFINITY;
            mloc = fmaxf(mloc, sc[kb][qb][r]);
          }
        // a column the chunk masks entirely keeps kNegBig: that chunk is the
        // wave's last, and its probabilities are exactly 0
        const float m0 = fmaxf(col_max_swap(mloc) * scale_log2, kNegBig);
        if (pass == 0) m_ref[qb] = m0;
        m_seen[qb] = m0;
      }
    }
    GL_STAMP(kKernFwd, 22);
    if (pass == 0 && q_rot != nullptr) {
      // q_rot as whole rows, issued after chunk 0's wait so that it does not
      // wait for these stores
#pragma unroll
      for (int n = 0; n < QI; ++n) {
        const int idx = tid + n * NT;
        const int r = idx / PPR, j = idx % PPR;
        if (r < nq) {
          const long gq = ((qrow0 + r) * n_heads_q + h) * D + 8 * j;
          store8(q_rot + gq, qy[n][0]);
          store8(q_rot + gq + H, qy[n][1]);
        }
      }
    }
    GL_STAMP(kKernFwd, 3);
    int i = 0;
    for (; i + 2 < nit; ++i) {
      iteration(i, std::true_type{}, std::false_type{}, std::true_type{});
      if (i < 6) GL_STAMP(kKernFwd, 5 + 2 * i);
    }
    if (i + 1 < nit) {
      iteration(i, std::true_type{}, std::true_type{}, std::false_type{});
      ++i;
    }
    GL_STAMP(kKernFwd, 16);
    if (i < nit) iteration(i, std::false_type{}, std::false_type{}, std::false_type{});
    fence_acc(o, lsum);
    GL_STAMP(kKernFwd, 17);
    if (__builtin_amdgcn_ballot_w64(grew) == 0) break;
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) m_seen[qb] = col_max_swap(m_seen[qb]);
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) m_ref[qb] = m_seen[qb];
  }
  GL_STAMP(kKernFwd, 20);

  // Merge.  Wave w < QB owns query block w.  Each wave writes its raw partial
  // O^T of the blocks it does not own and its (maximum, sum) per query into
  // its own ring region (free once its loop is done, so no wave waits for the
  // others first), straight from the AGPRs.  After one barrier each owner
  // weighs the four partials by exp2(m_u - M) / L (M = max of the maxima,
  // L = sum of exp2(m_u - M) l_u, both in wave order), adds them in wave
  // order (its own from registers) and stores its 16 rows.
  constexpr int MBLK = kFwdWaves > QB ? QB : QB - 1;  // blocks one wave writes, at most
  static_assert(MBLK * 16 * F::OS + 2 * TR <= F::WAVE / 2, "merge data exceeds a wave's region");
  float* const mine = reinterpret_cast<float*>(kring);  // [MBLK blocks][16][OS], maxima, sums
  constexpr int MOFF = MBLK * 16 * F::OS;                // maxima, then sums (floats)
  // the block slot of query block qb in the region of wave u (u does not own qb)
  auto slot_of = [](int u, int qb) { return u < QB ? qb - (qb > u) : qb; };
  if (g == 0) {
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      mine[MOFF + 16 * qb + c] = m_ref[qb];
      mine[MOFF + TR + 16 * qb + c] = lsum[qb][0];
    }
  }
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    if (qb == w) continue;
    const unsigned a = lds_addr(reinterpret_cast<const bf16*>(mine + (slot_of(w, qb) * 16 + c) * F::OS + 4 * g));
    write_acc_block(a, o, qb, std::make_integer_sequence<int, NDB>{});
  }
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the merge writes are complete
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  GL_STAMP(kKernFwd, 24);
  __syncthreads();
  GL_STAMP(kKernFwd, 25);
  if (w < QB) {
    const int qi = 16 * w + c;
    const float* region[kFwdWaves];
#pragma unroll
    for (int u = 0; u < kFwdWaves; ++u) region[u] = reinterpret_cast<const float*>(lds + u * F::WAVE);
    float mw[kFwdWaves], lw[kFwdWaves];
    float m_all = kNegBig;
#pragma unroll
    for (int u = 0; u < kFwdWaves; ++u) {
      mw[u] = region[u][MOFF + qi];
      lw[u] = region[u][MOFF + TR + qi];
      m_all = fmaxf(m_all, mw[u]);
    }
    float l_all = 0.0f;
#pragma unroll
    for (int u = 0; u < kFwdWaves; ++u) {
      mw[u] = __builtin_amdgcn_exp2f(mw[u] - m_all);
      l_all += lw[u] * mw[u];
    }
    const float inv = 1.0f / l_all;
    if (g == 0 && lse != nullptr && qi < nq)
      lse[(long)h * total_tokens + td.tok0 + q0 + qi] = (m_all + log2f(l_all)) * kLn2;
    f32x4 acc[NDB];
    // OWN: the owner's block as a constant (one branch on the wave index)
    auto sum_block = [&](auto own) {
      constexpr int OWN = decltype(own)::value;
#pragma unroll
      for (int db = 0; db < NDB; ++db) acc[db] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int u = 0; u < kFwdWaves; ++u) {
        const float f = mw[u] * inv;
#pragma unroll
        for (int db = 0; db < NDB; ++db) {
          const f32x4 x =
              u == OWN ? o[db][OWN]
                       : *reinterpret_cast<const f32x4*>(region[u] + (slot_of(u, OWN) * 16 + c) * F::OS +
                                                         16 * db + 4 * g);
          acc[db] += x * f;
        }
      }
    };
    if (w == 0) {
      sum_block(std::integral_constant<int, 0>{});
    } else if constexpr (QB == 1) {
    } else if (w == 1) {
      sum_block(std::integral_constant<int, 1>{});
    } else if constexpr (QB == 4) {
      if (w == 2)
        sum_block(std::integral_constant<int, 2>{});
      else
        sum_block(std::integral_constant<int, 3>{});
    }
    GL_STAMP(kKernFwd, 28);
    // rows of the block: lane (g, c) holds d = 16 db + 4 g .. + 3 of query qi
    if (qi < nq) {
      IO* const orow = out + ((qrow0 + qi) * n_heads_q + h) * D + 4 * g;
#pragma unroll
      for (int db = 0; db < NDB; ++db) store4(orow + 16 * db, acc[db]);
    }
  }
  GL_STAMP(kKernFwd, 21);
}

}  // namespace

template <typename IO, int D>
hipError_t launch_fwd_bf16(const FwdLaunch& a, hipStream_t st, KernelTimer* tm) {
  // 32-query workgroups (two per table entry) when the launch is short of CUs
  const int nsub = a.tile_rows == 16 ? 4 : a.tile_rows == 32 ? 2 : 1;  // workgroups per 64-row tile
  auto fn = a.single_seq ? attn_fwd_kernel_ks<IO, D, false, 4> : attn_fwd_kernel_ks<IO, D, true, 4>;
  if (nsub == 2) fn = a.single_seq ? attn_fwd_kernel_ks<IO, D, false, 2> : attn_fwd_kernel_ks<IO, D, true, 2>;
  if (nsub == 4) fn = a.single_seq ? attn_fwd_kernel_ks<IO, D, false, 1> : attn_fwd_kernel_ks<IO, D, true, 1>;
  constexpr size_t lds = FwdLayout<D>::BYTES;
  GL_CHECK(allow_lds(fn, lds));
  // the tables are one allocation: the sine table's offset in floats
  const ptrdiff_t sin_off = a.sin_t - a.cos_t;
  if (sin_off <= 0 || sin_off > INT32_MAX) return hipErrorInvalidValue;
  const int group = a.n_heads_q / a.n_heads_kv;
  LaunchTiming t(tm, kKernFwd);
  GL_LAUNCH(t, fn, dim3(group, a.n_heads_kv, a.n_tiles * nsub), dim3(kFwdWaves * 64), lds,
                        st, a.total_tokens, a.n_heads_kv, group, static_cast<int>(sin_off),
                        static_cast<const bf16*>(a.kc),
                        static_cast<const bf16*>(a.vc != nullptr ? a.vc : a.v), a.tiles_fwd,
                        static_cast<const IO*>(a.q), a.cos_t, static_cast<IO*>(a.out), a.lse,
                        static_cast<IO*>(a.q_rot), a.scale_log2);
  GL_CHECK(hipGetLastError());
  t.launched();
  return hipSuccess;
}

template hipError_t launch_fwd_bf16<bf16, 64>(const FwdLaunch&, hipStream_t, KernelTimer*);
template hipError_t launch_fwd_bf16<bf16, 128>(const FwdLaunch&, hipStream_t, KernelTimer*);
template hipError_t launch_fwd_bf16<float, 64>(const FwdLaunch&, hipStream_t, KernelTimer*);
template hipError_t launch_fwd_bf16<float, 128>(const FwdLaunch&, hipStream_t, KernelTimer*);

}  // namespace glacier

#ifdef GLACIER_PHASE_STAMPS
// Profiling builds only: copies this file's phase stamps (the forward's) to
// host memory.
extern "C" int glacier_attn_debug_stamps_fwd(void* host, size_t bytes) {
  return static_cast<int>(hipMemcpyFromSymbol(host, HIP_SYMBOL(glacier::glacier_stamps), bytes));
}
#endif
