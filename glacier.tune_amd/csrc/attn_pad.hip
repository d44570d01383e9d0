// attn_pad.hip -- head sizes the attention kernels are not built for.
//
// GpuLoraEngine.SupportsAttention (GpuLoraEngine.cs:111-112) takes any head
// size; the kernels are instantiated for 32, 64, 96, 128 and 256.  A call
// with another head size d runs them on copies of its rows padded to the
// next of those sizes, dp, laid out so that the rotation pairs
// (i, i + d/2) of RoPEKernel.cs:74-84 stay pairs of the padded row: the first
// half's d/2 elements go to columns 0 .. d/2 - 1, the second half's to
// dp/2 .. dp/2 + d/2 - 1, an odd d's last (unrotated) element to column d/2,
// and every other column is zero.  The engine's RoPE table for such a call
// holds the angles of d in its first d/2 columns and the identity rotation
// (cos 1, sin 0) after them, so padded columns stay zero (or keep the odd
// element) through every rotation, contribute nothing to a score or a row
// term, and come out of dQ/dK/dV as zeros; the softmax scale is that of d.
#include "attn_common.hpp"
#include "attn_launch.hpp"

namespace glacier {
namespace {

// The source column of padded column j (-1: a zero column).
__device__ inline int pad_source(int j, int d, int dp) {
  const int h = d / 2, hp = dp / 2;
  if (j < hp) {
    if (j < h) return j;
    return ((d & 1) && j == h) ? 2 * h : -1;
  }
  const int i = j - hp;
  return i < h ? h + i : -1;
}

// The padded column of source column s.
__device__ inline int pad_target(int s, int d, int dp) {
  const int h = d / 2, hp = dp / 2;
  if (s < h) return s;
  if (s < 2 * h) return hp + (s - h);
  return h;  // an odd d's last element
}

// one thread per padded element: dst[r][j] = src[r][pad_source(j)] or 0
template <typename T>
__global__ __launch_bounds__(256) void pad_rows_kernel(const T* __restrict__ src, T* __restrict__ dst,
                                                      long n, int d, int dp) {
  const long i = (long)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  const long r = i / dp;
  const int j = static_cast<int>(i - r * dp);
  const int s = pad_source(j, d, dp);
  dst[i] = s >= 0 ? src[r * d + s] : static_cast<T>(0.0f);
}

// one thread per source element: dst[r][s] = src[r][pad_target(s)]
template <typename T>
__global__ __launch_bounds__(256) void unpad_rows_kernel(const T* __restrict__ src, T* __restrict__ dst,
                                                        long n, int d, int dp) {
  const long i = (long)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  const long r = i / d;
  const int s = static_cast<int>(i - r * d);
  dst[i] = src[r * dp + pad_target(s, d, dp)];
}

template <typename T>
hipError_t launch_pad(const void* src, void* dst, long rows, int d, int dp, bool pad, hipStream_t st) {
  const long n = rows * (pad ? dp : d);
  if (n == 0) return hipSuccess;
  const dim3 grid(static_cast<unsigned>((n + 255) / 256));
  if (pad)
    hipLaunchKernelGGL(pad_rows_kernel<T>, grid, dim3(256), 0, st, static_cast<const T*>(src),
                       static_cast<T*>(dst), n, d, dp);
  else
    hipLaunchKernelGGL(unpad_rows_kernel<T>, grid, dim3(256), 0, st, static_cast<const T*>(src),
                       static_cast<T*>(dst), n, d, dp);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_pad_rows(bool io_bf16, const void* src, void* dst, long rows, int d, int dp,
                           hipStream_t st) {
  return io_bf16 ? launch_pad<bf16>(src, dst, rows, d, dp, true, st)
              : launch_pad<float>(src, dst, rows, d, dp, true, st);
}

hipError_t launch_unpad_rows(bool io_bf16, const void* src, void* dst, long rows, int d, int dp,
                             hipStream_t st) {
  return io_bf16 ? launch_pad<bf16>(src, dst, rows, d, dp, false, st)
              : launch_pad<float>(src, dst, rows, d, dp, false, st);
}

}  // namespace glacier
