/*
 * ce_oracle.c -- TEST INFRASTRUCTURE ONLY.
 *
 * CPU restatement of the LM-head cross-entropy loss and its gradient with
 * respect to the final hidden states, used as the parity checker for the
 * library's glacier_lmhead_* entry points.  Nothing in the product library
 * links or calls this file.
 *
 * It follows FusedCrossEntropyLoss (src/Glacier.Tune/Kernels/
 * FusedCrossEntropyLoss.cs; ComputeLoss :38-162, ComputeLossAndGradients
 * :170-364) loop for loop:
 *   rows whose target is outside [0, vocab) are dropped (:53, :190);
 *   vocab tiles of 4096 (:18): logits = hidden W_tile^T (:118, :268;
 *   QuantKernels.MatMulBatch for the F32 weight type, in the absent
 *   Glacier.Inference 1.8.0 package, restated as a dot product over k
 *   ascending); the target logit is picked up in its tile (:126, :276);
 *   a running max in float and a running sum of expf terms in double
 *   (:130-143, :280-293; VectorizedMax :382-434, VectorizedSumExp :436-444);
 *   loss = mean over the kept rows of (max + log(sum)) - target logit
 *   (:147-153, :297-302, :347: the sum in double, then (float)(total * 1/n));
 *   gradient pass (:304-345): the tile's logits recomputed, then
 *   dlogit = (exp(l - lse) - 1) / n at the target (in double, :327) and
 *   expf((float)(l - lse)) / n elsewhere, then LoraKernels.
 *   AccumulateBaseBackward (:336; F32 path, LoraKernels.BaseBackward.cs:39-74):
 *   dh[s][k] += dlogit[s][v] W[v][k] over v ascending, zero dlogits skipped;
 *   d_hidden is cleared (:183) and the kept rows' gradients scattered back
 *   (:346, ScatterValidGradients :367-378).
 * -ffp-contract=off (Makefile): C# float arithmetic has no implicit FMA.
 *
 * Layouts: hidden, d_hidden [T][H]; W [V][H] (GGUF row order); targets [T].
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#define CE_TILE 4096

/* logits[i][v] = sum_k h[i][k] W[v0 + v][k] for the tile [v0, v0 + nv). */
static void tile_logits(const float *h, const float *w, float *logits, int n, int H, int v0,
                        int nv) {
#pragma omp parallel for schedule(static)
  for (int i = 0; i < n; i++) {
    const float *hr = h + (size_t)i * H;
    for (int v = 0; v < nv; v++) {
      const float *wr = w + (size_t)(v0 + v) * H;
      float s = 0.0f;
      for (int k = 0; k < H; k++) s += hr[k] * wr[k];
      logits[(size_t)i * nv + v] = s;
    }
  }
}

/* Loss (returned) and, when d_hidden is not NULL, its gradient d_hidden [T][H]
 * (overwritten).  *n_valid receives the number of kept rows. */
float oracle_ce_loss(const float *hidden, const int *targets, const float *w, float *d_hidden,
                     int T, int H, int V, int *n_valid) {
  int *keep = (int *)malloc(sizeof(int) * (size_t)(T > 0 ? T : 1));
  int n = 0;
  for (int t = 0; t < T; t++)
    if (targets[t] >= 0 && targets[t] < V) keep[n++] = t;
  *n_valid = n;
  if (d_hidden != NULL) memset(d_hidden, 0, sizeof(float) * (size_t)T * H);
  if (n == 0) {
    free(keep);
    return 0.0f;
  }
  const float inv = 1.0f / (float)n;
  float *h = (float *)malloc(sizeof(float) * (size_t)n * H);
  float *g = (float *)calloc((size_t)n * H, sizeof(float));
  int *tgt = (int *)malloc(sizeof(int) * (size_t)n);
  for (int i = 0; i < n; i++) {
    memcpy(h + (size_t)i * H, hidden + (size_t)keep[i] * H, sizeof(float) * (size_t)H);
    tgt[i] = targets[keep[i]];
  }
  const int tile = V < CE_TILE ? V : CE_TILE;
  const int n_tiles = (V + tile - 1) / tile;
  float *logits = (float *)malloc(sizeof(float) * (size_t)n * tile);
  float *run_max = (float *)malloc(sizeof(float) * (size_t)n);
  double *run_sum = (double *)malloc(sizeof(double) * (size_t)n);
  float *tgt_logit = (float *)malloc(sizeof(float) * (size_t)n);
  double *lse = (double *)malloc(sizeof(double) * (size_t)n);
  for (int i = 0; i < n; i++) {
    run_max[i] = -INFINITY;
    run_sum[i] = 0.0;
    tgt_logit[i] = 0.0f;
  }
  for (int ti = 0; ti < n_tiles; ti++) {
    const int v0 = ti * tile, nv = (V - v0 < tile) ? V - v0 : tile;
    tile_logits(h, w, logits, n, H, v0, nv);
    for (int i = 0; i < n; i++) {
      const float *l = logits + (size_t)i * nv;
      if (tgt[i] >= v0 && tgt[i] < v0 + nv) tgt_logit[i] = l[tgt[i] - v0];
      float tmax = -INFINITY;
      for (int v = 0; v < nv; v++)
        if (l[v] > tmax) tmax = l[v];
      if (isinf(run_max[i]) && run_max[i] < 0) {
        run_max[i] = tmax;
        double s = 0.0;
        for (int v = 0; v < nv; v++) s += expf(l[v] - tmax);
        run_sum[i] = s;
      } else {
        const float m = run_max[i] > tmax ? run_max[i] : tmax;
        const double factor = exp((double)run_max[i] - m);
        double s = 0.0;
        for (int v = 0; v < nv; v++) s += expf(l[v] - m);
        run_sum[i] = run_sum[i] * factor + s;
        run_max[i] = m;
      }
    }
  }
  double total = 0.0;
  for (int i = 0; i < n; i++) {
    lse[i] = run_max[i] + log(run_sum[i]);
    total += lse[i] - tgt_logit[i];
  }
  if (d_hidden != NULL) {
    for (int ti = 0; ti < n_tiles; ti++) {
      const int v0 = ti * tile, nv = (V - v0 < tile) ? V - v0 : tile;
      if (n_tiles > 1) tile_logits(h, w, logits, n, H, v0, nv);
#pragma omp parallel for schedule(static)
      for (int i = 0; i < n; i++) {
        float *l = logits + (size_t)i * nv;
        for (int v = 0; v < nv; v++) {
          if (v0 + v == tgt[i])
            l[v] = (float)(exp(l[v] - lse[i]) - 1.0) * inv;
          else
            l[v] = expf((float)(l[v] - lse[i])) * inv;
        }
      }
#pragma omp parallel for schedule(static)
      for (int i = 0; i < n; i++) {
        float *gr = g + (size_t)i * H;
        const float *l = logits + (size_t)i * nv;
        for (int v = 0; v < nv; v++) {
          const float d = l[v];
          if (d == 0.0f) continue;
          const float *wr = w + (size_t)(v0 + v) * H;
          for (int k = 0; k < H; k++) gr[k] += d * wr[k];
        }
      }
    }
    for (int i = 0; i < n; i++)
      memcpy(d_hidden + (size_t)keep[i] * H, g + (size_t)i * H, sizeof(float) * (size_t)H);
  }
  free(keep); free(h); free(g); free(tgt); free(logits); free(run_max); free(run_sum);
  free(tgt_logit); free(lse);
  return (float)(total * inv);
}
