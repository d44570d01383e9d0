/*
 * norm_oracle.c -- TEST INFRASTRUCTURE ONLY.
 *
 * CPU restatement of the residual add and RMSNorm either side of the attention
 * sub-block, forward and backward, used as the parity checker for the
 * library's glacier_rmsnorm_* entry points.  Nothing in the product library
 * links or calls this file.
 *
 * The reference calls ElementwiseKernels.RMSNorm / RMSNormBackward and
 * TensorOps.Add from the Glacier.Tensor 1.1.0 package (namespace
 * Glacier.Tensor.Compute), which is absent from the reference tree, so the
 * arithmetic is restated from the published RMSNorm definition (Zhang and
 * Sennrich, 2019) in the GGUF convention the model's rms_norm_eps belongs to:
 *   r = 1 / sqrt(mean_i x_i^2 + eps),   y_i = (x_i * r) * w_i
 * and its exact gradient, with g_i = w_i dy_i:
 *   dx_i = r g_i - (r^3 / n) x_i sum_j g_j x_j,   dw_i += sum_rows dy_i x_i r.
 * Call sites it stands for (src/Glacier.Tune/Model/TransformerBlock.cs):
 *   forward   :318 norm1X = RMSNorm(x); :505-506 x1 = x + OProj(attnOut);
 *             :524 norm2X = RMSNorm(x1); :579 output = x1 + downOut (the next
 *             block's :318 then normalises it)
 *   backward  :672 RMSNormBackward(dNorm2X, X1) and :677 dX1 = dOutput + that;
 *             :827 RMSNormBackward(dNorm1X, x) and :836 dX = dX1 + that;
 *             :751, :759 the per-head Q/K norms (rows = tokens x heads)
 * Every call site passes null for the weight gradient (the norm weights are
 * frozen); d_weight is still restated for completeness.  Sums run over i
 * ascending in float; -ffp-contract=off (Makefile).
 *
 * Layouts: x, delta, x1, y, dy, d_residual, dx [rows][n]; w, d_weight [n].
 */
#include <math.h>
#include <stddef.h>

static float row_rstd(const float *x, int n, float eps) {
  float ss = 0.0f;
  for (int i = 0; i < n; i++) ss += x[i] * x[i];
  return 1.0f / sqrtf(ss / (float)n + eps);
}

/* x1 = x + delta (delta NULL: x1 = x; x1 may be NULL then), y = RMSNorm(x1) w. */
void oracle_rmsnorm_forward(const float *x, const float *delta, const float *w, float eps,
                            float *x1, float *y, int rows, int n) {
#pragma omp parallel for schedule(static)
  for (int t = 0; t < rows; t++) {
    const float *xr = x + (size_t)t * n;
    const float *src = xr;
    if (delta != NULL) {
      float *x1r = x1 + (size_t)t * n;
      const float *dr = delta + (size_t)t * n;
      for (int i = 0; i < n; i++) x1r[i] = xr[i] + dr[i];
      src = x1r;
    } else if (x1 != NULL) {
      float *x1r = x1 + (size_t)t * n;
      for (int i = 0; i < n; i++) x1r[i] = xr[i];
    }
    const float r = row_rstd(src, n, eps);
    float *yr = y + (size_t)t * n;
    for (int i = 0; i < n; i++) yr[i] = (src[i] * r) * w[i];
  }
}

/* dx = RMSNormBackward(dy; x, w) + d_residual (NULL: nothing added);
 * d_weight += sum over rows of dy x r (NULL: not formed). */
void oracle_rmsnorm_backward(const float *dy, const float *x, const float *w, float eps,
                             const float *d_residual, float *dx, float *d_weight, int rows,
                             int n) {
#pragma omp parallel for schedule(static)
  for (int t = 0; t < rows; t++) {
    const float *xr = x + (size_t)t * n, *dyr = dy + (size_t)t * n;
    const float r = row_rstd(xr, n, eps);
    float c = 0.0f;
    for (int i = 0; i < n; i++) c += (w[i] * dyr[i]) * xr[i];
    const float k = r * r * r / (float)n * c;
    float *dxr = dx + (size_t)t * n;
    for (int i = 0; i < n; i++) {
      float v = r * (w[i] * dyr[i]) - k * xr[i];
      if (d_residual != NULL) v += d_residual[(size_t)t * n + i];
      dxr[i] = v;
    }
  }
  if (d_weight == NULL) return;
  for (int t = 0; t < rows; t++) {
    const float *xr = x + (size_t)t * n, *dyr = dy + (size_t)t * n;
    const float r = row_rstd(xr, n, eps);
    for (int i = 0; i < n; i++) d_weight[i] += dyr[i] * (xr[i] * r);
  }
}
