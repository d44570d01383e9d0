/*
 * oracle_asan_driver.c -- runs every entry point of the CPU oracle
 * (oracle/*.c) under AddressSanitizer and UndefinedBehaviorSanitizer
 * (tests/test_sanitizers.py builds and runs it).  Every buffer is its own
 * exactly-sized heap block, so a read or write one element past what a
 * function may touch aborts the run.  Shapes cover the edges the parity tests
 * use: one-token sequences, partial tiles, empty segments in a packed batch,
 * every GQA ratio, head_dim 64 and 128, projections with and without bias and
 * adapters, RMSNorm with and without its optional operands, and a
 * cross-entropy over several vocabulary tiles with dropped rows.
 */
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

void oracle_rope_forward(float *q, float *k, int S, int Hq, int Hkv, int D, float freq_base,
                         float freq_scale, int rope_dim, const float *rope_freqs);
void oracle_rope_backward(float *dq, float *dk, int S, int Hq, int Hkv, int D, float freq_base,
                          float freq_scale, int rope_dim, const float *rope_freqs);
void oracle_rope_table(float *cs, float *sn, int S, int D, float freq_base);
void oracle_attn_forward_lse(const float *q, const float *k, const float *v, float *out,
                             float *probs, float *lse, int S, int Hq, int Hkv, int D);
int oracle_attn_backward(const float *dO, const float *q, const float *k, const float *v,
                         const float *probs, float *dq, float *dk, float *dv, int S, int Hq,
                         int Hkv, int D);
int oracle_layer_fwd_bwd(float *q, float *k, const float *v, const float *dO, float *out,
                         float *probs, float *lse, float *dq, float *dk, float *dv, int S, int Hq,
                         int Hkv, int D, float freq_base);
int oracle_layer_fwd_bwd_varlen(float *q, float *k, const float *v, const float *dO, float *out,
                                float *lse, float *dq, float *dk, float *dv, const int32_t *cu,
                                int n, int Hq, int Hkv, int D, float freq_base);
void oracle_fill_normal(float *x, size_t n, uint64_t seed, float mean, float std);
void oracle_proj_forward(const float *x, const float *w, const float *bias, const float *a,
                         const float *b, float scaling, float *y, int S, int in, int out,
                         int rank);
void oracle_proj_backward(const float *x, const float *dy, const float *w, const float *a,
                          const float *b, float scaling, float *dx, float *grad_a, float *grad_b,
                          int S, int in, int out, int rank);
void oracle_rmsnorm_forward(const float *x, const float *delta, const float *w, float eps,
                            float *x1, float *y, int rows, int n);
void oracle_rmsnorm_backward(const float *dy, const float *x, const float *w, float eps,
                             const float *d_residual, float *dx, float *d_weight, int rows, int n);
float oracle_ce_loss(const float *hidden, const int *targets, const float *w, float *d_hidden,
                     int T, int H, int V, int *n_valid);

static uint64_t g_seed = 1;

/* An exactly-sized block of n floats, filled with N(0, 1) (NULL for n == 0). */
static float *rnd(size_t n) {
  if (n == 0) return NULL;
  float *p = (float *)malloc(n * sizeof(float));
  if (p == NULL) abort();
  oracle_fill_normal(p, n, g_seed++, 0.0f, 1.0f);
  return p;
}

static float *out_buf(size_t n) {
  if (n == 0) return NULL;
  float *p = (float *)malloc(n * sizeof(float));
  if (p == NULL) abort();
  memset(p, 0xff, n * sizeof(float)); /* NaN: a skipped write shows up */
  return p;
}

static void attention_case(int S, int Hq, int Hkv, int D) {
  const size_t nq = (size_t)S * Hq * D, nk = (size_t)S * Hkv * D;
  float *q = rnd(nq), *k = rnd(nk), *v = rnd(nk), *dO = rnd(nq);
  float *out = out_buf(nq), *probs = out_buf((size_t)Hq * S * S), *lse = out_buf((size_t)Hq * S);
  float *dq = out_buf(nq), *dk = out_buf(nk), *dv = out_buf(nk);
  float *cs = out_buf((size_t)S * (D / 2)), *sn = out_buf((size_t)S * (D / 2));
  oracle_rope_table(cs, sn, S, D, 1.0e4f);
  oracle_rope_forward(q, k, S, Hq, Hkv, D, 1.0e4f, 1.0f, -1, NULL);
  oracle_attn_forward_lse(q, k, v, out, probs, lse, S, Hq, Hkv, D);
  if (oracle_attn_backward(dO, q, k, v, probs, dq, dk, dv, S, Hq, Hkv, D) != 0) abort();
  oracle_rope_backward(dq, dk, S, Hq, Hkv, D, 1.0e4f, 1.0f, -1, NULL);
  if (oracle_layer_fwd_bwd(q, k, v, dO, out, probs, lse, dq, dk, dv, S, Hq, Hkv, D, 1.0e6f) != 0)
    abort();
  free(q); free(k); free(v); free(dO); free(out); free(probs); free(lse);
  free(dq); free(dk); free(dv); free(cs); free(sn);
}

static void varlen_case(const int32_t *lens, int n, int Hq, int Hkv, int D) {
  int32_t *cu = (int32_t *)malloc(sizeof(int32_t) * (size_t)(n + 1));
  cu[0] = 0;
  for (int b = 0; b < n; b++) cu[b + 1] = cu[b] + lens[b];
  const int T = cu[n];
  const size_t nq = (size_t)T * Hq * D, nk = (size_t)T * Hkv * D;
  float *q = rnd(nq), *k = rnd(nk), *v = rnd(nk), *dO = rnd(nq);
  float *out = out_buf(nq), *lse = out_buf((size_t)Hq * T);
  float *dq = out_buf(nq), *dk = out_buf(nk), *dv = out_buf(nk);
  if (oracle_layer_fwd_bwd_varlen(q, k, v, dO, out, lse, dq, dk, dv, cu, n, Hq, Hkv, D, 1.0e6f) != 0)
    abort();
  free(cu); free(q); free(k); free(v); free(dO); free(out); free(lse);
  free(dq); free(dk); free(dv);
}

static void proj_case(int S, int in, int out, int rank, int with_bias) {
  float *x = rnd((size_t)S * in), *w = rnd((size_t)out * in), *dy = rnd((size_t)S * out);
  float *bias = with_bias ? rnd((size_t)out) : NULL;
  float *a = rank > 0 ? rnd((size_t)in * rank) : NULL, *b = rank > 0 ? rnd((size_t)rank * out) : NULL;
  float *y = out_buf((size_t)S * out), *dx = out_buf((size_t)S * in);
  float *ga = rank > 0 ? out_buf((size_t)in * rank) : NULL;
  float *gb = rank > 0 ? out_buf((size_t)rank * out) : NULL;
  if (ga != NULL) memset(ga, 0, (size_t)in * rank * sizeof(float));
  if (gb != NULL) memset(gb, 0, (size_t)rank * out * sizeof(float));
  oracle_proj_forward(x, w, bias, a, b, 0.5f, y, S, in, out, rank);
  oracle_proj_backward(x, dy, w, a, b, 0.5f, dx, ga, gb, S, in, out, rank);
  oracle_proj_backward(x, dy, w, a, b, 0.5f, NULL, ga, gb, S, in, out, rank);
  free(x); free(w); free(dy); free(bias); free(a); free(b); free(y); free(dx); free(ga); free(gb);
}

static void norm_case(int rows, int n, int with_delta, int with_residual, int with_dw) {
  float *x = rnd((size_t)rows * n), *w = rnd((size_t)n), *dy = rnd((size_t)rows * n);
  float *delta = with_delta ? rnd((size_t)rows * n) : NULL;
  float *dres = with_residual ? rnd((size_t)rows * n) : NULL;
  float *x1 = with_delta ? out_buf((size_t)rows * n) : NULL;
  float *y = out_buf((size_t)rows * n), *dx = out_buf((size_t)rows * n);
  float *dw = with_dw ? out_buf((size_t)n) : NULL;
  if (dw != NULL) memset(dw, 0, (size_t)n * sizeof(float));
  oracle_rmsnorm_forward(x, delta, w, 1e-6f, x1, y, rows, n);
  oracle_rmsnorm_backward(dy, x, w, 1e-6f, dres, dx, dw, rows, n);
  free(x); free(w); free(dy); free(delta); free(dres); free(x1); free(y); free(dx); free(dw);
}

static void ce_case(int T, int H, int V, int drop_every) {
  float *h = rnd((size_t)T * H), *w = rnd((size_t)V * H), *dh = out_buf((size_t)T * H);
  int *t = (int *)malloc(sizeof(int) * (size_t)(T > 0 ? T : 1));
  for (int i = 0; i < T; i++)
    t[i] = (drop_every > 0 && i % drop_every == 0) ? (i % 2 ? -1 : V) : (i * 7919) % V;
  int nv = -1;
  (void)oracle_ce_loss(h, t, w, dh, T, H, V, &nv);
  (void)oracle_ce_loss(h, t, w, NULL, T, H, V, &nv);
  free(h); free(w); free(dh); free(t);
}

int main(void) {
  const int shapes[][4] = {
      {1, 2, 1, 64}, {2, 4, 4, 128}, {17, 7, 1, 128}, {63, 4, 2, 64}, {65, 6, 3, 128}, {100, 8, 2, 64},
  };
  for (size_t i = 0; i < sizeof(shapes) / sizeof(shapes[0]); i++)
    attention_case(shapes[i][0], shapes[i][1], shapes[i][2], shapes[i][3]);
  const int32_t lens_a[] = {5, 0, 1, 70, 0};
  varlen_case(lens_a, 5, 4, 2, 64);
  const int32_t lens_b[] = {33, 64, 2};
  varlen_case(lens_b, 3, 14, 2, 128);
  proj_case(5, 32, 48, 4, 1);
  proj_case(3, 17, 9, 0, 0);
  proj_case(1, 64, 64, 8, 0);
  norm_case(4, 96, 1, 1, 1);
  norm_case(3, 33, 0, 0, 0);
  norm_case(1, 8, 1, 0, 1);
  ce_case(6, 40, 9000, 3);  /* three vocabulary tiles, dropped rows */
  ce_case(4, 16, 100, 0);
  ce_case(3, 8, 50, 1);     /* every row dropped */
  ce_case(0, 8, 50, 0);
  printf("ORACLE_SANITIZE_OK\n");
  return 0;
}
