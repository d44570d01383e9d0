/*
 * glacier_norm.h -- C ABI of the residual add and RMSNorm either side of the
 * attention sub-block in libglacier_attn.so, forward and backward, on device
 * tensors.  With glacier_proj_* (glacier_qkv.h) for the O projection and its
 * LoRA adapter, the whole path from the attention output to the FFN input,
 * and back, stays in HBM.
 *
 *   forward   x1 = x + delta,  y = RMSNorm(x1) weight
 *             (y_i = (x1_i r) weight_i,  r = 1 / sqrt(mean_i x1_i^2 + eps))
 *   backward  dx = RMSNormBackward(dy; x, weight) + d_residual
 *             (dx_i = r weight_i dy_i - (r^3 / n) x_i sum_j weight_j dy_j x_j)
 *
 * Replaces ElementwiseKernels.RMSNorm / RMSNormBackward and TensorOps.Add
 * (Glacier.Tensor 1.1.0) at the block's call sites
 * (src/Glacier.Tune/Model/TransformerBlock.cs):
 *   :318        norm1X = RMSNorm(x)                      forward, delta NULL
 *   :505-506    x1 = x + OProj(attnOut); :524 norm2X = RMSNorm(x1)
 *                                                        forward, delta = OProj output
 *   :579        output = x1 + downOut (normalised by the next block's :318)
 *                                                        forward, delta = downOut
 *   :672, :677  dX1 = dOutput + RMSNormBackward(dNorm2X, X1)
 *                                                        backward, d_residual = dOutput
 *   :827, :836  dX = dX1 + RMSNormBackward(dNorm1X, x)   backward, d_residual = dX1
 *   :751, :759  per-head Q/K norms in place (rows = tokens x heads, n = head_dim)
 *
 * Layouts (row-major): x, delta, x1, y, dy, d_residual, dx [rows][n] in the
 * io dtype; weight, d_weight [n] fp32.  Sums and the norm are fp32.  The
 * contexts, status codes and dtype constants are those of glacier_attn.h; calls
 * enqueue on the context's stream.
 */
#ifndef GLACIER_NORM_H
#define GLACIER_NORM_H

#include "glacier_attn.h"

#ifdef __cplusplus
extern "C" {
#endif

/* widest normalised row */
#define GLACIER_NORM_MAX_N 8192

typedef struct glacier_norm_desc {
  int32_t rows;      /* tokens, or tokens x heads for a per-head norm (may be 0) */
  int32_t n;         /* normalised width: a multiple of 4, at most GLACIER_NORM_MAX_N */
  int32_t io_dtype;  /* GLACIER_ATTN_IO_F32 or GLACIER_ATTN_IO_BF16 */
  float eps;         /* rms_norm_eps, finite and >= 0 */
} glacier_norm_desc;

/* x1 = x + delta and y = RMSNorm(x1) weight.  delta NULL: y = RMSNorm(x)
 * weight, and x1 is not written (may be NULL).  With delta, x1 is required
 * (the backward takes it as x); in the bf16 io dtype the norm is taken of x1
 * as stored.  y may alias x or delta; x1 may alias x. */
int glacier_rmsnorm_forward(glacier_attn_ctx *ctx, const glacier_norm_desc *desc, const void *x,
                            const void *delta, const float *weight, void *x1, void *y);

/* dx = RMSNormBackward(dy; x, weight) + d_residual (NULL: nothing added),
 * overwritten; x is the forward's normalised input (x1 there).  d_weight
 * (NULL: not formed, as at every reference call site) is accumulated (+=).
 * dx may alias dy or d_residual. */
int glacier_rmsnorm_backward(glacier_attn_ctx *ctx, const glacier_norm_desc *desc, const void *dy,
                             const void *x, const float *weight, const void *d_residual, void *dx,
                             float *d_weight);

#ifdef __cplusplus
}
#endif

#endif /* GLACIER_NORM_H */
