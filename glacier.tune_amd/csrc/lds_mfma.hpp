// lds_mfma.hpp -- pieces shared by the kernels that stage bf16 tiles in LDS
// by DMA and read them back from inline assembly for 32x32x16 MFMAs
// (attn_bwd3.hip, proj_gemm.hip): the row swizzle, LDS reads with immediate
// offsets and explicit waits, wave-uniform buffer resources.
//
// The compiler does not track LDS written by buffer_load ... lds, and its own
// LDS reads would make it wait for every load in flight, so the reads are
// issued from inline assembly and each kernel places its own s_waitcnt.
#pragma once

#include "attn_common.hpp"

#include <utility>

namespace glacier {

typedef float f32x16 __attribute__((ext_vector_type(16)));

// Slot of piece p of row r: p ^ lds_sw(r) (16 pieces per row at D = 128, 8 at
// D = 64, where two rows share one 256-byte line of the 64 banks).
template <int D>
__device__ inline int lds_sw(int r) {
  if constexpr (D == 128)
    return ((r & 3) << 2) | ((r >> 2) & 3);
  else
    return (((r >> 1) & 1) << 2) | ((r >> 2) & 3);
}

__device__ inline f32x4 lds4(unsigned addr) {
  f32x4 r;
  asm volatile("ds_read_b128 %0, %1" : "=v"(r) : "v"(addr));
  return r;
}
template <int OFF>
__device__ inline bf16x8 rd128(unsigned addr) {
  bf16x8 r;
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "i"(OFF));
  return r;
}
template <int OFF>
__device__ inline bf16x4 rdtr(unsigned addr) {
  bf16x4 r;
  asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "i"(OFF));
  return r;
}
template <int N>
__device__ inline void lgkm() {
  static_assert(N >= 0 && N < 16, "lgkmcnt range");
  asm volatile("s_waitcnt lgkmcnt(%0)" ::"i"(N) : "memory");
}
// lgkm<n> with n known only after unrolling (constant-folded there),
// saturated at the counter's maximum (a larger count waits for nothing)
__device__ inline void lgkm_v(int n) {
  switch (n < 15 ? n : 15) {
    case 0: lgkm<0>(); break;
    case 1: lgkm<1>(); break;
    case 2: lgkm<2>(); break;
    case 3: lgkm<3>(); break;
    case 4: lgkm<4>(); break;
    case 5: lgkm<5>(); break;
    case 6: lgkm<6>(); break;
    case 7: lgkm<7>(); break;
    case 8: lgkm<8>(); break;
    case 9: lgkm<9>(); break;
    case 10: lgkm<10>(); break;
    case 11: lgkm<11>(); break;
    case 12: lgkm<12>(); break;
    case 13: lgkm<13>(); break;
    case 14: lgkm<14>(); break;
    default: lgkm<15>(); break;
  }
}
template <int N>
__device__ inline void vmw() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0)" ::"i"(N) : "memory");
}
// vmcnt(n) for n known only after the call's arguments are (0 .. 63)
__device__ inline void vm_wait_v(int n) {
  switch (n) {
#define GL_VMW_CASE(N) \
  case N:              \
    vmw<N>();          \
    break;
    GL_VMW_CASE(0) GL_VMW_CASE(1) GL_VMW_CASE(2) GL_VMW_CASE(3) GL_VMW_CASE(4) GL_VMW_CASE(5)
    GL_VMW_CASE(6) GL_VMW_CASE(7) GL_VMW_CASE(8) GL_VMW_CASE(9) GL_VMW_CASE(10) GL_VMW_CASE(11)
    GL_VMW_CASE(12) GL_VMW_CASE(13) GL_VMW_CASE(14) GL_VMW_CASE(15) GL_VMW_CASE(16)
    GL_VMW_CASE(17) GL_VMW_CASE(18) GL_VMW_CASE(19) GL_VMW_CASE(20) GL_VMW_CASE(21)
    GL_VMW_CASE(22) GL_VMW_CASE(23) GL_VMW_CASE(24) GL_VMW_CASE(25) GL_VMW_CASE(26)
    GL_VMW_CASE(27) GL_VMW_CASE(28) GL_VMW_CASE(29) GL_VMW_CASE(30) GL_VMW_CASE(31)
    GL_VMW_CASE(32) GL_VMW_CASE(33) GL_VMW_CASE(34) GL_VMW_CASE(35) GL_VMW_CASE(36)
#undef GL_VMW_CASE
    default: vmw<0>(); break;
  }
}
// A workgroup barrier that waits for nothing itself: __syncthreads() is a
// release/acquire fence around s_barrier, and the compiler meets the fence by
// waiting for every DMA in flight (vmcnt(0)), which would drain the ring's
// prefetch at each step.  Callers wait for exactly what the barrier must
// order (vmw, lgkm) before it; the memory clobber keeps every memory access
// on its side.
__device__ inline void wg_barrier() { asm volatile("s_barrier" ::: "memory"); }

template <typename T>
__device__ inline void tie_v(T& x) {
  asm volatile("" : "+v"(x));
}
template <typename T>
__device__ inline T fresh_v(T x) {
  asm volatile("" : "+v"(x));
  return x;
}

__device__ inline bf16x8 join8(bf16x4 lo, bf16x4 hi) {
  bf16x8 r;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    r[i] = lo[i];
    r[4 + i] = hi[i];
  }
  return r;
}

// A buffer resource over [base, base + bytes) with base made wave-uniform.
#if defined(__HIP_DEVICE_COMPILE__)
__device__ inline __amdgpu_buffer_rsrc_t wave_rsrc(const void* base, int bytes) {
  const unsigned long long a = reinterpret_cast<unsigned long long>(base);
  const unsigned long long au =
      (static_cast<unsigned long long>(__builtin_amdgcn_readfirstlane(static_cast<int>(a >> 32))) << 32) |
      static_cast<unsigned>(__builtin_amdgcn_readfirstlane(static_cast<int>(a & 0xffffffffu)));
  return __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void*>(au), (short)0,
                                           __builtin_amdgcn_readfirstlane(bytes), kBufferWord3);
}
#endif

}  // namespace glacier
