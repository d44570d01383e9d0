// attn_ks.hpp -- building blocks of the LDS-DMA kernel (attn_fwd.hip):
// 32-row chunks of a [T][H][D] bf16 tensor copied from L2 straight into
// XOR-swizzled LDS tiles (buffer_load ... lds), LDS reads issued from inline
// assembly with explicit waits (the compiler ties its own forms of them to
// every outstanding DMA), and MFMAs whose accumulators are pinned in AGPRs.
#pragma once

#include "attn_common.hpp"

#include <utility>

namespace glacier {

constexpr int kChunk = 32;  // rows of one DMA chunk: one k-step of a bf16 MFMA

// Unpadded [rows][D] bf16 LDS tiles keep row r's 16-byte piece p in slot
// p ^ swz(r), so that the 16 rows read by one MFMA fragment (or by one
// transposing read) fall in distinct banks: rows of 256 B (D=128) each span
// all 64 banks, rows of 128 B (D=64) half of them, alternately.
template <int D>
__device__ inline int swz(int r) {
  return D == 128 ? (r & 15) : ((r >> 1) & 7);
}

// One 32-row chunk of a [T][H][D] bf16 tensor (the K or V rows of one head)
// into the swizzled LDS tile dst, by DMA (buffer_load ... lds, 16
// bytes per lane): instruction n fills 1 KB of dst, lane l the 16 bytes at
// l * 16, i.e. slot l % (D/8) of row n * (512/D) + l / (D/8).  The per-lane
// offsets repeat every P instructions (the swizzle period) and are computed
// once.  A chunk with fewer than 32 rows left in its sequence repeats row
// nvalid - 1 for the rest: those keys lie past every query of the sequence,
// so their probabilities are exactly 0 and any finite contents give the
// same sums.
// Completion is tracked by vmcnt only (the compiler does not track these
// writes): see wait_vmcnt.
// The per-lane part of the offsets, by instruction index modulo P.
struct DmaLanes {
  int rowb, rl, slot;
  int loff[4];
};

template <int D>
struct DmaShape {
  static constexpr int PPR = D / 8;           // 16-byte pieces per row
  static constexpr int RPI = 64 / PPR;        // rows per instruction
  static constexpr int NI = kChunk / RPI;     // instructions per chunk
  static constexpr int P = D == 128 ? 4 : 2;  // swizzle period in instructions
};

template <int D>
__device__ inline DmaLanes dma_lanes(long gstride, int lane) {
  using L = DmaShape<D>;
  DmaLanes dl;
  dl.rowb = __builtin_amdgcn_readfirstlane(static_cast<int>(gstride * (long)sizeof(bf16)));
  dl.rl = lane / L::PPR;
  dl.slot = lane % L::PPR;
#pragma unroll
  for (int n = 0; n < 4; ++n)
    dl.loff[n] = dl.rl * dl.rowb + 16 * (dl.slot ^ swz<D>((n % L::P) * L::RPI + dl.rl));
  return dl;
}

// (The body is compiled for the device only: instantiated in the host pass,
// the buffer-resource builtins invalidated the specialization for every
// later kernel instantiation, which then lost its launch stub.)
template <int D>
__device__ inline void dma_chunk(const DmaLanes& dl, const bf16* src, int nvalid, bf16* dst) {
#if defined(__HIP_DEVICE_COMPILE__)
  using L = DmaShape<D>;
  const unsigned long long a = reinterpret_cast<unsigned long long>(src);
  const unsigned long long au =
      (static_cast<unsigned long long>(__builtin_amdgcn_readfirstlane(static_cast<int>(a >> 32))) << 32) |
      static_cast<unsigned>(__builtin_amdgcn_readfirstlane(static_cast<int>(a & 0xffffffffu)));
  const int nv = __builtin_amdgcn_readfirstlane(nvalid < kChunk ? nvalid : kChunk);
  const __amdgpu_buffer_rsrc_t rs =
      __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void*>(au), (short)0, nv * dl.rowb, kBufferWord3);
  if (nv == kChunk) {
    // whole chunk: the row offset of instruction n goes into the scalar
    // offset (no per-lane arithmetic inside the loop)
#pragma unroll
    for (int n = 0; n < L::NI; ++n)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (GLACIER_LDS void*)(dst + 512 * n), 16, dl.loff[n % L::P],
                                               n * L::RPI * dl.rowb, 0, 0);
  } else {
    // lane row n RPI + rl loads row min(n RPI + rl, nv - 1), i.e. steps
    // min(n RPI, nv - 1 - rl) rows (the range check covers the vector
    // offset only, so the rows go there)
    const int limb = (nv - 1 - dl.rl) * dl.rowb;
#pragma unroll
    for (int n = 0; n < L::NI; ++n) {
      const int step = n * L::RPI * dl.rowb;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (GLACIER_LDS void*)(dst + 512 * n), 16,
                                               dl.loff[n % L::P] + (step < limb ? step : limb), 0, 0, 0);
    }
  }
#endif
}

// Waits until at most N vector-memory operations of this wave are
// outstanding; a compiler barrier keeps LDS reads of the chunk below it.
template <int N>
__device__ inline void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x0F70);  // expcnt, lgkmcnt: no wait
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// 32-bit LDS address of a pointer into dynamic shared memory.
__device__ inline unsigned lds_addr(const bf16* p) {
  return static_cast<unsigned>(reinterpret_cast<uintptr_t>((const GLACIER_LDS void*)p));
}

// ds_read_b64_tr_b16 issued from inline assembly: lane (g, i) addresses row
// R + i / 4 (R = the lane's row) at column c0 + 4 (i % 4) and receives rows
// R .. R + 3 of column c0 + i.  The compiler's own form of this read makes
// it wait for every outstanding LDS DMA of the wave (vmcnt(0)), i.e. for the
// next chunk's prefetch; these reads are ordered against the DMA by
// wait_vmcnt instead.  The result registers are valid only after wait_tr.
template <int OFF>
__device__ inline bf16x4 read_tr_async(unsigned addr) {
  bf16x4 r;
  asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "i"(OFF));
  return r;
}

// ds_read_b128 issued from inline assembly (K fragments, OFF: the offset
// field), valid after wait_kfrags<N>: LDS reads complete in order, so with
// N reads issued after the fragments, lgkmcnt(N) covers them.
template <int OFF>
__device__ inline bf16x8 read_b128_async(unsigned addr) {
  bf16x8 r;
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "i"(OFF));
  return r;
}
// s_waitcnt lgkmcnt(0) that the compiler sees as redefining the results of
// the preceding read_tr_async calls, so no use of them moves above it.
__device__ inline void wait_tr(bf16x4 (&t)[8]) {
  asm volatile("s_waitcnt lgkmcnt(0)"
               : "+v"(t[0]), "+v"(t[1]), "+v"(t[2]), "+v"(t[3]), "+v"(t[4]), "+v"(t[5]),
                 "+v"(t[6]), "+v"(t[7]));
}
__device__ inline void wait_tr(bf16x4 (&t)[16]) {
  asm volatile("s_waitcnt lgkmcnt(0)"
               : "+v"(t[0]), "+v"(t[1]), "+v"(t[2]), "+v"(t[3]), "+v"(t[4]), "+v"(t[5]),
                 "+v"(t[6]), "+v"(t[7]), "+v"(t[8]), "+v"(t[9]), "+v"(t[10]), "+v"(t[11]),
                 "+v"(t[12]), "+v"(t[13]), "+v"(t[14]), "+v"(t[15]));
}

// acc += A B (v_mfma_f32_16x16x32_bf16) with the accumulator pinned in
// AGPRs: the O^T tiles stay in place across the loop instead of being
// copied between register files.  The compiler does not see an MFMA here,
// so the asm itself provides the two wait states a VALU-written operand
// needs (s_nop 1), and fence_acc below the MFMA-to-reader wait states.
__device__ inline void mma_acc(f32x4& acc, const bf16x8& a, const bf16x8& b) {
  asm("s_nop 1\n\tv_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b));
}
// Two independent accumulations behind one pair of wait states (one issue
// slot fewer than two mma_acc calls).
__device__ inline void mma_acc2(f32x4& acc0, const bf16x8& a0, const bf16x8& b0, f32x4& acc1,
                                const bf16x8& a1, const bf16x8& b1) {
  asm("s_nop 1\n\tv_mfma_f32_16x16x32_bf16 %0, %2, %3, %0\n\tv_mfma_f32_16x16x32_bf16 %1, %4, %5, %1"
      : "+a"(acc0), "+a"(acc1)
      : "v"(a0), "v"(b0), "v"(a1), "v"(b1));
}

// ds_write_b128 of an accumulator straight from its AGPRs (OFF: the offset
// field, bytes).  Use after fence_acc; completion is waited for explicitly.
template <int OFF>
__device__ inline void write_acc(unsigned addr, const f32x4& v) {
  asm volatile("ds_write_b128 %0, %1 offset:%2" : : "v"(addr), "a"(v), "i"(OFF) : "memory");
}

}  // namespace glacier
