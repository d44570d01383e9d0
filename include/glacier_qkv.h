/*
 * glacier_qkv.h -- C ABI of the projection step either side of attention in
 * libglacier_attn.so: the frozen base projections of one normalised input
 * plus their trainable LoRA adapters, forward and backward, on device
 * tensors, so that Q, K and V go from the projection into attention (and
 * dQ, dK, dV back) without leaving HBM.
 *
 * For each projection p (q, k and v in a transformer block):
 *   forward   Y_p = X W_p^T + bias_p + s_p (X A_p) B_p
 *   backward  dX  = sum_p dY_p W_p + s_p (dY_p B_p^T) A_p^T
 *             grad_A_p += s_p X^T (dY_p B_p^T),  grad_B_p += s_p (X A_p)^T dY_p
 * Replaces GpuLoraEngine.ForwardQKV (GpuLoraEngine.Forward.cs:205-245),
 * which runs the base GEMMs on the GPU, copies Q/K/V to the host and adds
 * the LoRA deltas there (AddLoraDeltaHost, :366-399, i.e.
 * LoraKernels.ApplyLoraDelta, LoraKernels.cs:18-122), and the three
 * LoraAdapter.Backward calls of the block (LoraAdapter.cs:190-247:
 * LoraKernels.AccumulateBaseBackward, LoraKernels.BaseBackward.cs:21-75,
 * then LoraKernels.Backward, LoraKernels.cs:125-345).  s_p is the adapter's
 * alpha / rank (LoraAdapter.cs:98); the base weights are frozen.
 *
 * Layouts (row-major): x, dx [T][in]; w [out][in] (GGUF row order);
 * bias [out]; lora_a [in][rank]; lora_b [rank][out]; y, dy [T][out].
 * x, w, y, dy and dx have the call's io dtype; bias, the adapters and their
 * gradients are fp32.  The contexts, status codes and dtype constants are
 * those of glacier_attn.h; calls enqueue on the context's stream.
 */
#ifndef GLACIER_QKV_H
#define GLACIER_QKV_H

#include "glacier_attn.h"

#ifdef __cplusplus
extern "C" {
#endif

/* largest LoRA rank and number of projections per call */
#define GLACIER_PROJ_MAX_RANK 64
#define GLACIER_PROJ_MAX_PROJ 4

/* One projection of the call's input. */
typedef struct glacier_lora_proj {
  const void *w;         /* [out][in] base weight (io dtype) */
  const float *bias;     /* [out], or NULL */
  const float *lora_a;   /* [in][rank], or NULL for no adapter */
  const float *lora_b;   /* [rank][out] (required with lora_a) */
  float scaling;         /* alpha / rank */
  int32_t out_features;  /* a multiple of 4 */
  void *y;               /* forward: [T][out] output, overwritten */
  const void *dy;        /* backward: [T][out] upstream gradient */
  float *grad_a;         /* backward: [in][rank], accumulated (+=); may be NULL */
  float *grad_b;         /* backward: [rank][out], accumulated (+=); may be NULL */
} glacier_lora_proj;

typedef struct glacier_proj_desc {
  int32_t total_tokens;  /* T (may be 0) */
  int32_t in_features;   /* a multiple of 4 */
  int32_t rank;          /* 1..GLACIER_PROJ_MAX_RANK when any adapter is given */
  int32_t precision;     /* GLACIER_ATTN_PREC_*: FP32 (fp32 GEMMs) or BF16 */
  int32_t io_dtype;      /* GLACIER_ATTN_IO_*: F32, or BF16 with PREC_BF16 (bf16
                            GEMM operands, fp32 accumulation and adapters) */
} glacier_proj_desc;

/* Forward of n_proj (1..GLACIER_PROJ_MAX_PROJ) projections of x.  Each y is
 * overwritten; outputs must not alias inputs. */
int glacier_proj_forward(glacier_attn_ctx *ctx, const glacier_proj_desc *desc,
                         const void *x, const glacier_lora_proj *proj, int n_proj);

/* Backward of the same projections: dx [T][in] is overwritten with the sum
 * over p of the base and adapter gradients (what the reference's three
 * LoraAdapter.Backward calls accumulate into a zeroed dXInput); grad_a and
 * grad_b are accumulated, like the reference's Grad tensors. */
int glacier_proj_backward(glacier_attn_ctx *ctx, const glacier_proj_desc *desc,
                          const void *x, const glacier_lora_proj *proj, int n_proj,
                          void *dx);

#ifdef __cplusplus
}
#endif

#endif /* GLACIER_QKV_H */
