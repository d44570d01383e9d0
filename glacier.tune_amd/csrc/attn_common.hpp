// attn_common.hpp -- device-side building blocks shared by the attention
// kernels (gfx950, wave64).
//
// Matrix-core conventions.  Every product in this library is a 16x16 MFMA
// tile, D[16x16] += A[16xK] * B[Kx16], with one of
//   bf16: v_mfma_f32_16x16x32_bf16  (K = 32, 8 bf16 of k per lane)
//   fp32: v_mfma_f32_16x16x4_f32    (K = 4, 1 float of k per lane)
// Lane l (g = l / 16, c = l % 16) supplies A[row c][k = KPL*g .. +KPL-1] and
// B[k = KPL*g .. +KPL-1][col c], and receives D[row 4g + r][col c], r = 0..3.
//
// Scores are computed transposed where a wave owns 16 queries (S^T = K Q^T,
// queries as the MFMA columns) and plainly where it owns 16 keys (S = Q K^T,
// keys as the columns), so a lane's accumulators always belong to ONE column
// (one query, or one key) and hold 4 consecutive rows 16b + 4g + r of each
// 16-row block b.  Those registers are fed straight back as the B operand of
// the next product (O^T += V^T P^T, dQ^T += K^T dS^T, dV^T += dO^T P,
// dK^T += Q^T dS) by permuting the k index of the MFMA: for bf16 the 8
// k-slots of lane group g in 32-row step s are rows {32s + 4g + r} U
// {32s + 16 + 4g + r}.  The matching A operand is read from a ROW-MAJOR LDS
// tile with the gfx950 transpose read ds_read_b64_tr_b16: in each group of
// 16 lanes, lane 4a+b addresses row R + a, columns c0 + 4b .. +3, and lane i
// receives rows R .. R+3 of column c0 + i -- exactly the 4 consecutive rows
// the permuted k-slots want.  No tile is ever stored transposed, in LDS or
// in HBM.  Row statistics (max, sum, alpha) never leave the lane except for
// one xor-16/xor-32 exchange, and no accumulator is ever shuffled.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "attn_launch.hpp"

namespace glacier {

// f(integral_constant<int, i>) for i = 0 .. N - 1, in order
template <int N, typename F, int... I>
__device__ inline void static_for_impl(F&& f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}
template <int N, typename F>
__device__ inline void static_for(F&& f) {
  static_for_impl<N>(f, std::make_integer_sequence<int, N>{});
}


using bf16 = __bf16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef int i32x4 __attribute__((ext_vector_type(4)));

// Word 3 of a raw buffer resource on gfx9-family GPUs: 32-bit data format
// (a zero format would make every load return 0), no swizzle, no stride.
constexpr int kBufferWord3 = 0x00020000;

#define GLACIER_LDS __attribute__((address_space(3)))

template <typename T>
struct Mfma;

template <>
struct Mfma<bf16> {
  static constexpr int KPL = 8;
  static constexpr int KSTEP = 32;
  using Frag = bf16x8;
  __device__ static inline f32x4 mma(Frag a, Frag b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
};

template <>
struct Mfma<float> {
  static constexpr int KPL = 1;
  static constexpr int KSTEP = 4;
  using Frag = float;
  __device__ static inline f32x4 mma(Frag a, Frag b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
  }
};

// Row stride (elements) of a row-major [64][D] LDS tile, padded so the 16
// rows read by one MFMA operand fall in different banks: bf16 rows of 288 B
// (D=128) or 144 B (D=64), fp32 rows of D+4 floats.  (Measured on gfx950 for
// the 16-byte fragment reads: 148 B/clk/CU at 288 B against 104 at 272 B.)
template <typename T, int D>
struct Lds {
  static constexpr int CE = 16 / sizeof(T);  // elements per 16-byte chunk
  static constexpr int STRIDE = (sizeof(T) == 2 && D == 128) ? D + 2 * CE : D + CE;
  static constexpr int TILE = kTile * STRIDE;  // elements of one tile
};

__device__ inline float to_f32(float x) { return x; }
__device__ inline float to_f32(bf16 x) { return (float)x; }

template <typename T>
__device__ inline T from_f32(float x);
template <>
__device__ inline float from_f32<float>(float x) { return x; }
template <>
__device__ inline bf16 from_f32<bf16>(float x) { return (bf16)x; }

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
// 16 bytes from src (any address space) to global dst with the nontemporal
// hint (global_store_dwordx4 ... nt): the line is streamed out as it is
// written instead of staying dirty in the XCD's L2 until the end-of-kernel
// write-back.  For results no later work of the same kernel reads.
__device__ inline void store16_nt(void* dst, const void* src) {
  typedef unsigned u32x4_nt __attribute__((ext_vector_type(4)));
  __builtin_nontemporal_store(*reinterpret_cast<const u32x4_nt*>(src), reinterpret_cast<u32x4_nt*>(dst));
}
__device__ inline void store4(bf16* p, f32x4 v) {
  bf16x4 b;
#pragma unroll
  for (int i = 0; i < 4; ++i) b[i] = (bf16)v[i];
  *reinterpret_cast<bf16x4*>(p) = b;
}

// This thread's share of a [ROWS][D] tile (64 rows, or a 32-row key chunk)
// held in registers between a global load and an LDS store (the software
// pipeline of every kernel's main loop).  Chunks are 8 consecutive elements
// of one row; chunk index tid + i*NT maps to (row, chunk) with the chunk
// fastest, so a wave reads whole rows.
template <typename IO, int D, int NT = kThreads, int ROWS = kTile>
struct TileRegs {
  static constexpr int CPR = D / 8;                  // chunks per row
  // Lanes per row: CPR rounded up to a power of two, so that a row's lanes
  // never straddle a wave (D = 96: 12 chunks on 16 lanes, 4 of them idle
  // and holding zeros).
  static constexpr int LPR = CPR <= 4 ? 4 : CPR <= 8 ? 8 : CPR <= 16 ? 16 : 32;
  static constexpr int N = ROWS * LPR / NT;          // chunks per thread
  static constexpr int W = 8 * sizeof(IO) / 16;      // 16-byte words per chunk
  static_assert(CPR <= LPR && D % 8 == 0, "head_dim a multiple of 8, at most 256");
  static_assert(N * NT == ROWS * LPR, "tile must split evenly");
  i32x4 w[N][W];

  // Rows r >= nvalid read as zero (past the end of the sequence): the loads
  // go through a buffer resource whose range ends with row nvalid - 1, and
  // the hardware returns 0 for offsets beyond it.  Full and partial tiles
  // share one branch-free code path.  (With a separate bounds-checked path
  // writing the same registers, the compiler has to drain each tile's loads
  // before issuing the next tile's, serialising the memory round trips.)
  // src, gstride and nvalid must be uniform over the wave (they are read
  // from its first lane).
  __device__ inline void load(const IO* src, long gstride, int nvalid, int tid) {
    const int rowb = __builtin_amdgcn_readfirstlane(static_cast<int>(gstride * (long)sizeof(IO)));
    const int nv = nvalid < ROWS ? nvalid : ROWS;
    const int nrec = __builtin_amdgcn_readfirstlane(
        nv <= 0 ? 0 : (nv - 1) * rowb + D * static_cast<int>(sizeof(IO)));
    const unsigned long long a = reinterpret_cast<unsigned long long>(src);
    const unsigned long long au =
        (static_cast<unsigned long long>(__builtin_amdgcn_readfirstlane(static_cast<int>(a >> 32))) << 32) |
        static_cast<unsigned>(__builtin_amdgcn_readfirstlane(static_cast<int>(a & 0xffffffffu)));
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        reinterpret_cast<void*>(au), (short)0, nrec, kBufferWord3);
#pragma unroll
    for (int i = 0; i < N; ++i) {
      const int idx = tid + i * NT;
      const int r = idx / LPR, ch = idx % LPR;
      const int off = r * rowb + ch * 8 * static_cast<int>(sizeof(IO));
      if (LPR != CPR && ch >= CPR) {
#pragma unroll
        for (int j = 0; j < W; ++j) w[i][j] = i32x4{0, 0, 0, 0};
        continue;
      }
#pragma unroll
      for (int j = 0; j < W; ++j) w[i][j] = __builtin_amdgcn_raw_buffer_load_b128(rs, off + 16 * j, 0, 0);
    }
  }

  // Writes the tile to a row-major LDS tile of element type T (converting).
  template <typename T>
  __device__ inline void store(T* lds, int tid) const {
    constexpr int S = Lds<T, D>::STRIDE;
#pragma unroll
    for (int i = 0; i < N; ++i) {
      const int idx = tid + i * NT;
      const int r = idx / LPR, ch = idx % LPR;
      if (LPR != CPR && ch >= CPR) continue;
      T* dst = lds + r * S + ch * 8;
      if constexpr (sizeof(IO) == sizeof(T)) {
#pragma unroll
        for (int j = 0; j < W; ++j) reinterpret_cast<i32x4*>(dst)[j] = w[i][j];
      } else {
        float x[8];
        load8(reinterpret_cast<const IO*>(&w[i][0]), x);
        store8(dst, x);
      }
    }
  }
};

// A/B fragment from a row-major LDS tile: row `row`, k-step kk, lane group g.
template <typename T, int D>
__device__ inline typename Mfma<T>::Frag frag_rm(const T* lds, int row, int kk, int g) {
  using M = Mfma<T>;
  const T* p = lds + row * Lds<T, D>::STRIDE + kk * M::KSTEP + M::KPL * g;
  if constexpr (sizeof(T) == 2) {
    return *reinterpret_cast<const bf16x8*>(p);
  } else {
    return *p;
  }
}

// A/B fragment straight from a global row (token-major tensor), converted to
// the compute dtype: elements kk*KSTEP + KPL*g .. of the row.
template <typename T, typename IO>
__device__ inline typename Mfma<T>::Frag frag_global(const IO* rowp, int kk, int g) {
  using M = Mfma<T>;
  const IO* p = rowp + kk * M::KSTEP + M::KPL * g;
  if constexpr (sizeof(T) == 2) {
    if constexpr (sizeof(IO) == 2) {
      return *reinterpret_cast<const bf16x8*>(p);
    } else {
      float x[8];
      load8(p, x);
      bf16x8 f;
#pragma unroll
      for (int e = 0; e < 8; ++e) f[e] = (bf16)x[e];
      return f;
    }
  } else {
    return to_f32(*p);
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

// Transpose read: 4 consecutive rows R..R+3 of column c0 + (lane % 16) of a
// row-major bf16 LDS tile, where R = row0 + 4 * (lane / 16).
template <int STRIDE>
__device__ inline bf16x4 read_tr(const bf16* tile, int row0, int c0, int lane) {
  const int g = lane >> 4, i = lane & 15;
  const bf16* p = tile + (row0 + 4 * g + (i >> 2)) * STRIDE + c0 + 4 * (i & 3);
  return __builtin_amdgcn_ds_read_tr16_b64_v4bf16(
      (bf16x4 GLACIER_LDS*)(const_cast<bf16*>(p)));
}

// acc[db] (+)= sum over the 64 rows of the row-major LDS tile `tile`, of
// tile[row][16*db + i] * v[row-slot] -- i.e. Out^T[d][col] += Tile^T * V
// with Out^T row d = 16*db + i (the MFMA A row) and the lane's own values
// v[b][r] for row 16b + 4g + r as the B operand (permuted k-slots, see the
// top of this file).  Row blocks b >= nb are zero and skipped.
template <typename T, int D>
__device__ inline void acc_rows(f32x4 (&acc)[D / 16], const T* tile,
                                const float (&v)[4][4], int nb, int lane) {
  constexpr int S = Lds<T, D>::STRIDE;
  const int g = lane >> 4, c = lane & 15;
  if constexpr (sizeof(T) == 2) {
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      if (2 * s >= nb) break;
      bf16x8 bfrag;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        bfrag[r] = (bf16)v[2 * s][r];
        bfrag[4 + r] = (bf16)v[2 * s + 1][r];
      }
#pragma unroll
      for (int db = 0; db < D / 16; ++db) {
        const bf16x4 lo = read_tr<S>(tile, 32 * s, 16 * db, lane);
        const bf16x4 hi = read_tr<S>(tile, 32 * s + 16, 16 * db, lane);
        bf16x8 a;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          a[r] = lo[r];
          a[4 + r] = hi[r];
        }
        acc[db] = Mfma<bf16>::mma(a, bfrag, acc[db]);
      }
    }
  } else {
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      if (b >= nb) break;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
#pragma unroll
        for (int db = 0; db < D / 16; ++db) {
          const float a = tile[(16 * b + 4 * g + r) * S + 16 * db + c];
          acc[db] = Mfma<float>::mma(a, v[b][r], acc[db]);
        }
      }
    }
  }
}

// RoPE, written without contraction so that q_rot/k_rot are the exact fp32
// results of RoPEKernel.cs:84-85 (v0*c - v1*s, v0*s + v1*c) given the same
// cos/sin table.
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

// Phase timestamps for profiling builds (-DGLACIER_PHASE_STAMPS, see
// build.py --stamps): thread 0 of a workgroup records the wall clock (100 MHz)
// at named points of a kernel into glacier_stamps[kernel][workgroup][slot]
// (one array per source file: each has its own device code object);
// GL_STAMP_VALUE records a plain value (which tile the workgroup took).  In
// the product build both expand to nothing.
#ifdef GLACIER_PHASE_STAMPS
constexpr int kStampKernels = 4, kStampBlocks = 4096, kStampSlots = 32;
static __device__ unsigned long long glacier_stamps[kStampKernels][kStampBlocks][kStampSlots];
__device__ inline void phase_stamp(int kernel, int slot, unsigned long long value) {
  if (threadIdx.x == 0) {
    const unsigned b = (blockIdx.z * gridDim.y + blockIdx.y) * gridDim.x + blockIdx.x;
    if (b < kStampBlocks) glacier_stamps[kernel][b][slot] = value;
  }
}
#define GL_STAMP(kernel, slot) ::glacier::phase_stamp(kernel, slot, wall_clock64())
#define GL_STAMP_VALUE(kernel, slot, v) ::glacier::phase_stamp(kernel, slot, (v))
#else
#define GL_STAMP(kernel, slot) ((void)0)
#define GL_STAMP_VALUE(kernel, slot, v) ((void)0)
#endif

// Index of this wave in the workgroup, as a scalar: the compiler cannot
// prove threadIdx.x / 64 uniform, and values derived from it (the group's
// tile, its base pointers) must live in scalar registers to form buffer
// resources without a per-lane loop.
__device__ inline int wave_id() {
  return __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> 6);
}

// s_waitcnt vmcnt(0): wait for every outstanding vector-memory access of
// this wave (expcnt and lgkmcnt fields at their maxima, i.e. not waited on).
// Issued at the end of a kernel prologue it tells the compiler's wait
// tracking that the prologue's conditional loads (operand fragments kept in
// registers for the whole loop) are complete on every path; otherwise it
// guards their first use inside the loop with a wait that also drains the
// loop's own prefetch loads.
__device__ inline void wait_vmem_all() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// Sum over groups of N (4, 8, 16 or 32) consecutive lanes: DPP lane moves
// (quad xor 1, quad xor 2, half-row mirror, row mirror) run at ALU speed;
// only N = 32 needs one cross-row permute.  Every lane of a group ends with
// the same bits (each step adds two equal-order partial sums).
template <int N>
__device__ inline float lanes_sum(float x) {
  static_assert(N == 4 || N == 8 || N == 16 || N == 32, "4-, 8-, 16- or 32-lane groups");
  // (the DPP control operand must be a literal)
  x += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0xB1, 0xF, 0xF, false));
  x += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x4E, 0xF, 0xF, false));
  if constexpr (N == 4) return x;
  x += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x141, 0xF, 0xF, false));
  if constexpr (N >= 16)
    x += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x140, 0xF, 0xF, false));
  if constexpr (N == 32) x += __shfl_xor(x, 16);
  return x;
}

// Max / sum over the 4 lanes that share a column (lanes l, l^16, l^32,
// l^48) with the gfx950 lane-swap instructions: v_permlane32_swap of a value
// with itself leaves each lane one operand from its own half and one from
// the other, v_permlane16_swap likewise for the two rows of a half; no LDS
// traffic and no wait.  For the sum both lanes of a pair add the same two
// operands in the same order, so every lane gets the same bits.
__device__ inline float swap_max(float x, bool rows16) {
  const unsigned u = __builtin_bit_cast(unsigned, x);
  const auto r = rows16 ? __builtin_amdgcn_permlane16_swap(u, u, false, false)
                        : __builtin_amdgcn_permlane32_swap(u, u, false, false);
  const unsigned a = r[0], b = r[1];
  return fmaxf(__builtin_bit_cast(float, a), __builtin_bit_cast(float, b));
}
__device__ inline float swap_sum(float x, bool rows16) {
  const unsigned u = __builtin_bit_cast(unsigned, x);
  const auto r = rows16 ? __builtin_amdgcn_permlane16_swap(u, u, false, false)
                        : __builtin_amdgcn_permlane32_swap(u, u, false, false);
  const unsigned a = r[0], b = r[1];
  return __builtin_bit_cast(float, a) + __builtin_bit_cast(float, b);
}
__device__ inline float col_max_swap(float x) { return swap_max(swap_max(x, false), true); }
__device__ inline float col_sum_swap(float x) { return swap_sum(swap_sum(x, false), true); }

// Sum over the 4 lanes that share a column (xor 16, xor 32), in a fixed
// order so every lane gets the same bits.
__device__ inline float col_sum(float x) {
  x = x + __shfl_xor(x, 16);
  return x + __shfl_xor(x, 32);
}
__device__ inline float col_max(float x) {
  x = fmaxf(x, __shfl_xor(x, 16));
  return fmaxf(x, __shfl_xor(x, 32));
}

}  // namespace glacier
