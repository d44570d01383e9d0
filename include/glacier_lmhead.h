/*
 * glacier_lmhead.h -- C ABI of the LM-head cross-entropy loss and its
 * gradient with respect to the final hidden states in libglacier_attn.so, on
 * device tensors.
 *
 *   logits = hidden W^T                      (W [vocab][hidden], GGUF row order)
 *   loss   = mean over rows whose target is in [0, vocab) of
 *            logsumexp(logits[t]) - logits[t][target[t]]
 *   d_hidden[t] = (softmax(logits[t]) - onehot(target[t])) W / n_valid,
 *                 and 0 for rows whose target is outside [0, vocab)
 *
 * Replaces FusedCrossEntropyLoss.ComputeLoss and ComputeLossAndGradients
 * (src/Glacier.Tune/Kernels/FusedCrossEntropyLoss.cs:38-162, :170-364) and
 * their GPU tiles (GpuLoraEngine.ComputeTiledLmHeadLoss, GpuLoraEngine.
 * Backward.cs:98-197, and ComputeTiledLmHeadLossAndGradients, :203-352),
 * which stream 4096-wide vocabulary tiles through a host-side softmax.  Here
 * the logits stay in HBM (in chunks of at most 2 GB) and never reach the
 * host; the loss comes back as one float.
 *
 * The targets are a host array, as in the reference (int[] targetTokens);
 * the tensors are device pointers with the call's io dtype.  The contexts,
 * status codes and dtype constants are those of glacier_attn.h.  The calls
 * return when the loss is on the host (they synchronise the context's
 * stream).
 */
#ifndef GLACIER_LMHEAD_H
#define GLACIER_LMHEAD_H

#include "glacier_attn.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct glacier_lmhead_desc {
  int32_t tokens;     /* rows of hidden (may be 0) */
  int32_t hidden;     /* hidden size, a multiple of 8 */
  int32_t vocab;      /* vocabulary size, >= 1 */
  int32_t precision;  /* GLACIER_ATTN_PREC_FP32 or _BF16 */
  int32_t io_dtype;   /* GLACIER_ATTN_IO_F32 (fp32 GEMMs), or _BF16 with PREC_BF16
                         (bf16 GEMM operands, fp32 logits, softmax and accumulation) */
} glacier_lmhead_desc;

/* The mean cross-entropy (FusedCrossEntropyLoss.ComputeLoss).  targets: host
 * int32 [tokens]; *loss gets the mean (0 when no row is kept) and, if not
 * NULL, *n_valid the number of kept rows. */
int glacier_lmhead_loss(glacier_attn_ctx *ctx, const glacier_lmhead_desc *desc, const void *hidden,
                        const int32_t *targets, const void *weight, float *loss,
                        int32_t *n_valid);

/* The loss and d_hidden [tokens][hidden] (overwritten), as
 * FusedCrossEntropyLoss.ComputeLossAndGradients. */
int glacier_lmhead_loss_and_grad(glacier_attn_ctx *ctx, const glacier_lmhead_desc *desc,
                                 const void *hidden, const int32_t *targets, const void *weight,
                                 void *d_hidden, float *loss, int32_t *n_valid);

#ifdef __cplusplus
}
#endif

#endif /* GLACIER_LMHEAD_H */
