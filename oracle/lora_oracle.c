/*
 * lora_oracle.c -- TEST INFRASTRUCTURE ONLY.
 *
 * CPU restatement of the projection step either side of attention: a frozen
 * base projection plus a trainable LoRA adapter, forward and backward, used
 * as the parity checker for the library's glacier_proj_* entry points.
 * Nothing in the product library links or calls this file.
 *
 * It follows, loop for loop and in the same accumulation order:
 *   forward  LoraAdapter.Forward (src/Glacier.Tune/Model/LoraAdapter.cs:128-183):
 *     the base projection y[s][o] = sum_k x[s][k] W[o][k] (QuantKernels.MatMulBatch
 *     for the F32 weight type, :139; that kernel belongs to the Glacier.Inference
 *     1.8.0 package, which is absent, so it is restated here as a dot product
 *     over k ascending), the bias (:141-150), then LoraKernels.ApplyLoraDelta
 *     (src/Glacier.Tune/Kernels/LoraKernels.cs:18-122, the generic path of
 *     :88-115): lowRank = x A, then out += (lowRank * scaling) B with rows
 *     whose scaled value is exactly 0 skipped.
 *   backward LoraAdapter.Backward (LoraAdapter.cs:190-220, then :225-247): the base gradient
 *     LoraKernels.AccumulateBaseBackward, F32 path
 *     (src/Glacier.Tune/Kernels/LoraKernels.BaseBackward.cs:39-74:
 *     dx[s][k] += dy[s][o] W[o][k] over o ascending, zero dy skipped), then
 *     LoraKernels.Backward (LoraKernels.cs:125-345, generic paths): lowRank,
 *     gradB[r][n] += (lowRank[s][r] * scaling) dy[s][n] over s ascending,
 *     dLowRank = dy B^T over n ascending, gradA[k][r] += scaling * sum_s
 *     x[s][k] dLowRank[s][r], dx[s][k] += scaling * sum_r dLowRank[s][r] A[k][r].
 * The reference's AVX fast path for rank 16 uses fused multiply-adds and
 * differs from these loops only by rounding.  -ffp-contract=off (Makefile):
 * C# float arithmetic has no implicit FMA.
 *
 * Layouts: x, dx [S][in]; W [out][in] (the GGUF row order); bias [out];
 * A [in][rank]; B [rank][out]; y, dy [S][out].
 */
#include <stdlib.h>
#include <string.h>

/* lowRank[s][r] = sum_k x[s][k] A[k][r] (LoraKernels.cs:90-101, 170-185). */
static void low_rank(const float *x, const float *a, float *lr, int S, int in, int rank) {
#pragma omp parallel for schedule(static)
  for (int s = 0; s < S; s++) {
    const float *row = x + (size_t)s * in;
    for (int r = 0; r < rank; r++) {
      float sum = 0.0f;
      for (int k = 0; k < in; k++) sum += row[k] * a[(size_t)k * rank + r];
      lr[(size_t)s * rank + r] = sum;
    }
  }
}

/* y = x W^T + bias + scaling (x A) B.  a == NULL: no adapter. */
void oracle_proj_forward(const float *x, const float *w, const float *bias, const float *a,
                         const float *b, float scaling, float *y, int S, int in, int out,
                         int rank) {
#pragma omp parallel for schedule(static)
  for (int s = 0; s < S; s++) {
    const float *row = x + (size_t)s * in;
    for (int o = 0; o < out; o++) {
      const float *wr = w + (size_t)o * in;
      float sum = 0.0f;
      for (int k = 0; k < in; k++) sum += row[k] * wr[k];
      y[(size_t)s * out + o] = sum;
    }
    if (bias != NULL)
      for (int o = 0; o < out; o++) y[(size_t)s * out + o] += bias[o];
  }
  if (a == NULL || b == NULL || rank <= 0 || scaling == 0.0f) return;
  float *lr = (float *)malloc(sizeof(float) * (size_t)S * rank);
  low_rank(x, a, lr, S, in, rank);
#pragma omp parallel for schedule(static)
  for (int s = 0; s < S; s++) {                             /* LoraKernels.cs:103-112 */
    float *yr = y + (size_t)s * out;
    for (int r = 0; r < rank; r++) {
      float v = lr[(size_t)s * rank + r] * scaling;
      if (v == 0.0f) continue;
      const float *br = b + (size_t)r * out;
      for (int n = 0; n < out; n++) yr[n] += v * br[n];
    }
  }
  free(lr);
}

/* dx += dy W + scaling (dy B^T) A^T; grad_a += scaling x^T (dy B^T);
 * grad_b += scaling (x A)^T dy.  dx, grad_a, grad_b accumulate, as the
 * reference's Grad tensors and dXInput do; any of them may be NULL. */
void oracle_proj_backward(const float *x, const float *dy, const float *w, const float *a,
                          const float *b, float scaling, float *dx, float *grad_a,
                          float *grad_b, int S, int in, int out, int rank) {
  if (dx != NULL) {
#pragma omp parallel for schedule(static)
    for (int s = 0; s < S; s++) {                           /* BaseBackward.cs:62-72 */
      float *dxr = dx + (size_t)s * in;
      const float *dyr = dy + (size_t)s * out;
      for (int o = 0; o < out; o++) {
        float d = dyr[o];
        if (d == 0.0f) continue;
        const float *wr = w + (size_t)o * in;
        for (int k = 0; k < in; k++) dxr[k] += d * wr[k];
      }
    }
  }
  if (a == NULL || b == NULL || rank <= 0) return;
  float *lr = (float *)malloc(sizeof(float) * (size_t)S * rank);
  float *dlr = (float *)malloc(sizeof(float) * (size_t)S * rank);
  low_rank(x, a, lr, S, in, rank);                          /* LoraKernels.cs:145-185 */
  if (grad_b != NULL) {
#pragma omp parallel for schedule(static)
    for (int r = 0; r < rank; r++) {                        /* LoraKernels.cs:189-215 */
      float *gb = grad_b + (size_t)r * out;
      for (int s = 0; s < S; s++) {
        float v = lr[(size_t)s * rank + r] * scaling;
        const float *dyr = dy + (size_t)s * out;
        for (int n = 0; n < out; n++) gb[n] += v * dyr[n];
      }
    }
  }
#pragma omp parallel for schedule(static)
  for (int s = 0; s < S; s++) {                             /* LoraKernels.cs:218-246 */
    const float *dyr = dy + (size_t)s * out;
    for (int r = 0; r < rank; r++) {
      const float *br = b + (size_t)r * out;
      float dot = 0.0f;
      for (int n = 0; n < out; n++) dot += dyr[n] * br[n];
      dlr[(size_t)s * rank + r] = dot;
    }
  }
  if (grad_a != NULL) {
#pragma omp parallel for schedule(static)
    for (int k = 0; k < in; k++) {                          /* LoraKernels.cs:276-290 */
      float *ga = grad_a + (size_t)k * rank;
      for (int r = 0; r < rank; r++) {
        float sum = 0.0f;
        for (int s = 0; s < S; s++) sum += x[(size_t)s * in + k] * dlr[(size_t)s * rank + r];
        ga[r] += sum * scaling;
      }
    }
  }
  if (dx != NULL) {
#pragma omp parallel for schedule(static)
    for (int s = 0; s < S; s++) {                           /* LoraKernels.cs:322-337 */
      const float *dr = dlr + (size_t)s * rank;
      float *dxr = dx + (size_t)s * in;
      for (int k = 0; k < in; k++) {
        float dot = 0.0f;
        for (int r = 0; r < rank; r++) dot += dr[r] * a[(size_t)k * rank + r];
        dxr[k] += dot * scaling;
      }
    }
  }
  free(lr);
  free(dlr);
}
