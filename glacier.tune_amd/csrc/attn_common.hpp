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
// The kernels compute scores transposed, S^T = K Q^T (one wave owns 16
// queries as the MFMA columns), so a lane's accumulators all belong to ONE
// query (column c) and hold 4 consecutive keys 16b + 4g + r of each 16-key
// block b.  Those registers are fed straight back as the B operand of the
// next product (O^T += V^T P^T, dQ^T += K^T dS^T, dV^T += dO^T P, dK^T +=
// Q^T dS) by permuting the k index of the MFMA: for bf16 the 8 k-slots of
// lane group g in 32-key step s are keys {32s + 4g + r} U {32s + 16 + 4g + r};
// the A operand is read from a transposed LDS tile with the same map (two
// 8-byte reads).  Row statistics (max, sum, alpha) therefore never leave the
// lane except for one xor-16/xor-32 exchange, and no accumulator is ever
// shuffled.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "attn_launch.hpp"

namespace glacier {

using bf16 = __bf16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));


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

// LDS row strides (elements).  Row-major tiles: D + one 16-byte chunk, so
// the 16 rows read by one MFMA operand fall in different banks.
// Transposed tiles (64 columns): 64 + one 16-byte chunk.
template <typename T, int D>
struct Lds {
  static constexpr int CE = 16 / sizeof(T);  // elements per 16-byte chunk
  static constexpr int RM = D + CE;
  static constexpr int TR = kTile + CE;
  static constexpr int RM_ELEMS = kTile * RM;  // one row-major tile
  static constexpr int TR_ELEMS = D * TR;      // one transposed tile
};

__device__ inline float to_f32(float x) { return x; }
__device__ inline float to_f32(bf16 x) { return (float)x; }

template <typename T>
__device__ inline T from_f32(float x);
template <>
__device__ inline float from_f32<float>(float x) { return x; }
template <>
__device__ inline bf16 from_f32<bf16>(float x) { return (bf16)x; }

// 16-byte chunk copy global -> LDS, zero when `valid` is false.
template <typename T>
__device__ inline void copy16(T* dst, const T* src, bool valid) {
  uint4 v = valid ? *reinterpret_cast<const uint4*>(src) : make_uint4(0, 0, 0, 0);
  *reinterpret_cast<uint4*>(dst) = v;
}

// Stage a row-major [64][D] tile: rows r < nvalid come from src + r*gstride.
template <typename T, int D>
__device__ inline void stage_rm(T* lds, const T* src, long gstride, int nvalid,
                                int tid) {
  using L = Lds<T, D>;
  constexpr int CPR = D / L::CE;                // chunks per row
  constexpr int ITERS = kTile * CPR / kThreads;
#pragma unroll
  for (int it = 0; it < ITERS; ++it) {
    int idx = tid + it * kThreads;
    int r = idx / CPR, ch = idx % CPR;
    copy16(lds + r * L::RM + ch * L::CE, src + (long)r * gstride + ch * L::CE,
           r < nvalid);
  }
}

// Stage a transposed [D][64] tile: row d comes from src + d*gstride (64
// contiguous, 16-byte aligned, zero-padded columns).
template <typename T, int D>
__device__ inline void stage_tr(T* lds, const T* src, long gstride, int tid) {
  using L = Lds<T, D>;
  constexpr int CPR = kTile / L::CE;
  constexpr int ITERS = D * CPR / kThreads;
#pragma unroll
  for (int it = 0; it < ITERS; ++it) {
    int idx = tid + it * kThreads;
    int r = idx / CPR, ch = idx % CPR;
    copy16(lds + r * L::TR + ch * L::CE, src + (long)r * gstride + ch * L::CE,
           true);
  }
}

// A-operand fragment from a row-major LDS tile: row `row`, k-step kk.
template <typename T, int D>
__device__ inline typename Mfma<T>::Frag frag_rm(const T* lds, int row, int kk,
                                                 int g) {
  using M = Mfma<T>;
  const T* p = lds + row * Lds<T, D>::RM + kk * M::KSTEP + M::KPL * g;
  if constexpr (sizeof(T) == 2) {
    return *reinterpret_cast<const bf16x8*>(p);
  } else {
    return *p;
  }
}

// acc[db] (+)= sum over the 64 columns of the transposed tile `tt`
// (rows d = 16*db + c) times the lane's own probabilities/gradients
// v[b][r] (column 16b + 4g + r), i.e. Out^T += Tt * V^T with the permuted
// k-slot map described at the top of this file.  Blocks b >= nb are zero
// and skipped.
template <typename T, int D>
__device__ inline void acc_tr(f32x4 (&acc)[D / 16], const T* tt,
                              const float (&v)[4][4], int nb, int lane) {
  using L = Lds<T, D>;
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
        const T* row = tt + (16 * db + c) * L::TR + 32 * s + 4 * g;
        bf16x4 lo = *reinterpret_cast<const bf16x4*>(row);
        bf16x4 hi = *reinterpret_cast<const bf16x4*>(row + 16);
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
          float a = tt[(16 * db + c) * L::TR + 16 * b + 4 * g + r];
          acc[db] = Mfma<float>::mma(a, v[b][r], acc[db]);
        }
      }
    }
  }
}

// Sum over the 4 lanes that share a query/key column (xor 16, xor 32), in a
// fixed order so every lane gets the same bits.
__device__ inline float col_sum(float x) {
  x = x + __shfl_xor(x, 16);
  return x + __shfl_xor(x, 32);
}
__device__ inline float col_max(float x) {
  x = fmaxf(x, __shfl_xor(x, 16));
  return fmaxf(x, __shfl_xor(x, 32));
}

}  // namespace glacier
