/*
 * attn_oracle.c -- TEST INFRASTRUCTURE ONLY.
 *
 * CPU restatement of Glacier.Tune's causal grouped-query attention path, used
 * as the parity checker for the HIP kernels and as the timed CPU baseline
 * ("port") in bench.py.  Nothing in the product library links or calls this
 * file; only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg
 * load it.
 *
 * It follows, loop for loop and in the same accumulation order:
 *   src/Glacier.Tune/Kernels/RoPEKernel.cs:12-105            (rope_* below)
 *   src/Glacier.Tune/Kernels/CausalAttentionKernel.cs:17-77  (oracle_attn_forward)
 *   src/Glacier.Tune/Kernels/CausalAttentionKernel.cs:79-213 (oracle_attn_backward)
 * The reference is C#: MathF.Exp/Pow/Sin/Cos are taken to be the C runtime's
 * expf/powf/sinf/cosf, and C# float arithmetic is plain IEEE binary32 with no
 * implicit FMA, hence -ffp-contract=off and no -ffast-math in oracle/Makefile.
 * Parallel.For over heads becomes an OpenMP loop over heads; each head is
 * independent and the KV-group reduction runs in ascending head order, so the
 * thread count never changes a result bit.
 *
 * Extensions that the reference does not have (each pinned by its own tests):
 *   - oracle_attn_forward_lse: the same forward, also returning the row
 *     log-sum-exp lse[h][i] = max_i + logf(sumExp_i), the statistic the GPU
 *     path saves instead of P.  Pinned against fp64 closed forms.
 *   - oracle_attn_*_varlen: packed sequences with a block-diagonal causal
 *     mask; each segment is run through the single-sequence functions on its
 *     own rows, positions restarting at 0 (no reference counterpart; the
 *     reference is batch 1).
 *
 * Layouts (CausalAttentionKernel.cs:33,40): q/out/dO/dq are [S][Hq][D],
 * k/v/dk/dv are [S][Hkv][D], probs is [Hq][S][S]; kv head = h / (Hq/Hkv).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

/* RoPEKernel.cs:43-105 ApplyRoPE for one position. */
static void apply_rope_pos(float *q, float *k, int Hq, int Hkv, int D, int pos,
                           float freq_base, float freq_scale, int inverse,
                           int rope_dim, const float *rope_freqs) {
  int eff = (rope_dim > 0 && rope_dim <= D) ? rope_dim : D;  /* :53 */
  int half = eff / 2;
  if (half <= 0) return;
  float *cs = (float *)malloc(sizeof(float) * (size_t)half * 2);
  float *sn = cs + half;
  float sign = inverse ? -1.0f : 1.0f;
  for (int i = 0; i < half; i++) {                         /* :62-69 */
    float base_freq = 1.0f / powf(freq_base, (float)(2 * i) / (float)eff);
    float freq = rope_freqs ? (base_freq / rope_freqs[i]) : base_freq;
    float theta = (float)pos * freq * freq_scale;
    cs[i] = cosf(theta);
    sn[i] = sinf(theta) * sign;
  }
  for (int h = 0; h < Hq; h++) {                           /* :74-87 */
    float *hd = q + (size_t)h * D;
    for (int i = 0; i < half; i++) {
      float c = cs[i], s = sn[i], v0 = hd[i], v1 = hd[i + half];
      hd[i] = v0 * c - v1 * s;
      hd[i + half] = v0 * s + v1 * c;
    }
  }
  for (int h = 0; h < Hkv; h++) {                          /* :90-103 */
    float *hd = k + (size_t)h * D;
    for (int i = 0; i < half; i++) {
      float c = cs[i], s = sn[i], v0 = hd[i], v1 = hd[i + half];
      hd[i] = v0 * c - v1 * s;
      hd[i + half] = v0 * s + v1 * c;
    }
  }
  free(cs);
}

/* RoPEKernel.cs:12-25 ForwardSequence (serial over positions, like the reference). */
void oracle_rope_forward(float *q, float *k, int S, int Hq, int Hkv, int D,
                         float freq_base, float freq_scale, int rope_dim,
                         const float *rope_freqs) {
  for (int pos = 0; pos < S; pos++)
    apply_rope_pos(q + (size_t)pos * Hq * D, k + (size_t)pos * Hkv * D, Hq, Hkv,
                   D, pos, freq_base, freq_scale, 0, rope_dim, rope_freqs);
}

/* RoPEKernel.cs:27-41 BackwardSequence: same rotation with -sin. */
void oracle_rope_backward(float *dq, float *dk, int S, int Hq, int Hkv, int D,
                          float freq_base, float freq_scale, int rope_dim,
                          const float *rope_freqs) {
  for (int pos = 0; pos < S; pos++)
    apply_rope_pos(dq + (size_t)pos * Hq * D, dk + (size_t)pos * Hkv * D, Hq,
                   Hkv, D, pos, freq_base, freq_scale, 1, rope_dim, rope_freqs);
}

/* The per-position cos/sin table exactly as RoPEKernel.cs:62-69 computes it
 * (freqScale 1, no ropeFreqs); cs/sn are [S][D/2]. */
void oracle_rope_table(float *cs, float *sn, int S, int D, float freq_base) {
  int half = D / 2;
  for (int pos = 0; pos < S; pos++)
    for (int i = 0; i < half; i++) {
      float base_freq = 1.0f / powf(freq_base, (float)(2 * i) / (float)D);
      float theta = (float)pos * base_freq * 1.0f;
      cs[(size_t)pos * half + i] = cosf(theta);
      sn[(size_t)pos * half + i] = sinf(theta);
    }
}

/* CausalAttentionKernel.cs:17-77, plus lse (NULL = not wanted). */
void oracle_attn_forward_lse(const float *q, const float *k, const float *v,
                             float *out, float *probs, float *lse, int S,
                             int Hq, int Hkv, int D) {
  int ratio = Hq / Hkv;                                    /* :23 */
  float scale = 1.0f / sqrtf((float)D);                    /* :24 */
#pragma omp parallel for schedule(dynamic, 1)
  for (int h = 0; h < Hq; h++) {                           /* :26 */
    int kvh = h / ratio;
    float *ph = probs + (size_t)h * S * S;
    for (int i = 0; i < S; i++) {
      const float *qv = q + ((size_t)i * Hq + h) * D;
      float *prow = ph + (size_t)i * S;
      float mx = -INFINITY;
      for (int j = 0; j <= i; j++) {                       /* :38-46 */
        const float *kv = k + ((size_t)j * Hkv + kvh) * D;
        float sc = 0.0f;
        for (int d = 0; d < D; d++) sc += qv[d] * kv[d];
        sc *= scale;
        prow[j] = sc;
        if (sc > mx) mx = sc;
      }
      for (int j = i + 1; j < S; j++) prow[j] = 0.0f;      /* :49 */
      float sum = 0.0f;
      for (int j = 0; j <= i; j++) {                       /* :52-58 */
        float e = expf(prow[j] - mx);
        prow[j] = e;
        sum += e;
      }
      float inv = sum > 0.0f ? 1.0f / sum : 0.0f;          /* :59 */
      for (int j = 0; j <= i; j++) prow[j] *= inv;         /* :60 */
      if (lse) lse[(size_t)h * S + i] = mx + logf(sum);
      float *ov = out + ((size_t)i * Hq + h) * D;          /* :63-74 */
      for (int d = 0; d < D; d++) ov[d] = 0.0f;
      for (int j = 0; j <= i; j++) {
        float p = prow[j];
        const float *vv = v + ((size_t)j * Hkv + kvh) * D;
        for (int d = 0; d < D; d++) ov[d] += p * vv[d];
      }
    }
  }
}

void oracle_attn_forward(const float *q, const float *k, const float *v,
                         float *out, float *probs, int S, int Hq, int Hkv,
                         int D) {
  oracle_attn_forward_lse(q, k, v, out, probs, NULL, S, Hq, Hkv, D);
}

/* CausalAttentionKernel.cs:79-213.  Returns 0, or -1 if the workspace could
 * not be allocated. */
int oracle_attn_backward(const float *dO, const float *q, const float *k,
                         const float *v, const float *probs, float *dq,
                         float *dk, float *dv, int S, int Hq, int Hkv, int D) {
  int ratio = Hq / Hkv;
  float scale = 1.0f / sqrtf((float)D);
  memset(dq, 0, sizeof(float) * (size_t)S * Hq * D);      /* :90-92 */
  memset(dk, 0, sizeof(float) * (size_t)S * Hkv * D);
  memset(dv, 0, sizeof(float) * (size_t)S * Hkv * D);
  size_t per_head = (size_t)S * D;                         /* :95-98 */
  float *wsk = (float *)calloc((size_t)Hq * per_head, sizeof(float));
  float *wsv = (float *)calloc((size_t)Hq * per_head, sizeof(float));
  if (!wsk || !wsv) { free(wsk); free(wsv); return -1; }
#pragma omp parallel for schedule(dynamic, 1)
  for (int h = 0; h < Hq; h++) {                           /* :102 */
    int kvh = h / ratio;
    const float *ph = probs + (size_t)h * S * S;
    float *hdk = wsk + (size_t)h * per_head;
    float *hdv = wsv + (size_t)h * per_head;
    float *dp = (float *)malloc(sizeof(float) * (size_t)S * 2);
    float *ds = dp + S;
    for (int i = 0; i < S; i++) {                          /* :122 */
      const float *dov = dO + ((size_t)i * Hq + h) * D;
      const float *prow = ph + (size_t)i * S;
      float dot = 0.0f;
      for (int j = 0; j <= i; j++) {                       /* :129-136 */
        const float *vv = v + ((size_t)j * Hkv + kvh) * D;
        float acc = 0.0f;
        for (int d = 0; d < D; d++) acc += dov[d] * vv[d];
        dp[j] = acc;
        dot += prow[j] * acc;
      }
      for (int j = 0; j <= i; j++)                         /* :139-142 */
        ds[j] = prow[j] * (dp[j] - dot) * scale;
      float *dqv = dq + ((size_t)i * Hq + h) * D;          /* :145-154 */
      for (int j = 0; j <= i; j++) {
        float s = ds[j];
        const float *kv = k + ((size_t)j * Hkv + kvh) * D;
        for (int d = 0; d < D; d++) dqv[d] += s * kv[d];
      }
      const float *qv = q + ((size_t)i * Hq + h) * D;      /* :157-171 */
      for (int j = 0; j <= i; j++) {
        float s = ds[j], p = prow[j];
        float *a = hdk + (size_t)j * D;
        float *b = hdv + (size_t)j * D;
        for (int d = 0; d < D; d++) {
          a[d] += s * qv[d];
          b[d] += p * dov[d];
        }
      }
    }
    free(dp);
  }
#pragma omp parallel for schedule(static)
  for (int kvh = 0; kvh < Hkv; kvh++) {                    /* :184-206 */
    int h0 = kvh * ratio, h1 = h0 + ratio;
    for (int j = 0; j < S; j++) {
      float *dkd = dk + ((size_t)j * Hkv + kvh) * D;
      float *dvd = dv + ((size_t)j * Hkv + kvh) * D;
      for (int h = h0; h < h1; h++) {
        const float *sk = wsk + ((size_t)h * S + j) * D;
        const float *sv = wsv + ((size_t)h * S + j) * D;
        for (int d = 0; d < D; d++) {
          dkd[d] += sk[d];
          dvd[d] += sv[d];
        }
      }
    }
  }
  free(wsk);
  free(wsv);
  return 0;
}

/* The whole reference CPU layer path, TransformerBlock.cs:444-485 (forward)
 * and :731-741 (backward): RoPE forward in place on q/k, attention forward
 * into out/probs/lse, attention backward, RoPE backward on dq/dk.  q and k
 * come back post-RoPE, like the saved state (TransformerBlock.cs:490-497). */
int oracle_layer_fwd_bwd(float *q, float *k, const float *v, const float *dO,
                         float *out, float *probs, float *lse, float *dq,
                         float *dk, float *dv, int S, int Hq, int Hkv, int D,
                         float freq_base) {
  oracle_rope_forward(q, k, S, Hq, Hkv, D, freq_base, 1.0f, -1, NULL);
  oracle_attn_forward_lse(q, k, v, out, probs, lse, S, Hq, Hkv, D);
  int rc = oracle_attn_backward(dO, q, k, v, probs, dq, dk, dv, S, Hq, Hkv, D);
  if (rc) return rc;
  oracle_rope_backward(dq, dk, S, Hq, Hkv, D, freq_base, 1.0f, -1, NULL);
  return 0;
}

/* Packed variable-length batch: cu[0..n] are token offsets; segment b holds
 * rows cu[b]..cu[b+1]-1 of the token-major tensors; positions restart at 0.
 * probs is per segment [Hq][L][L], packed back to back; lse is [Hq][T]. */
int oracle_layer_fwd_bwd_varlen(float *q, float *k, const float *v,
                                const float *dO, float *out, float *lse,
                                float *dq, float *dk, float *dv,
                                const int32_t *cu, int n, int Hq, int Hkv,
                                int D, float freq_base) {
  int T = cu[n];
  for (int b = 0; b < n; b++) {
    int r0 = cu[b], L = cu[b + 1] - cu[b];
    if (L <= 0) continue;
    float *probs = (float *)malloc(sizeof(float) * (size_t)Hq * L * L);
    float *slse = (float *)malloc(sizeof(float) * (size_t)Hq * L);
    if (!probs || !slse) { free(probs); free(slse); return -1; }
    int rc = oracle_layer_fwd_bwd(
        q + (size_t)r0 * Hq * D, k + (size_t)r0 * Hkv * D,
        v + (size_t)r0 * Hkv * D, dO + (size_t)r0 * Hq * D,
        out + (size_t)r0 * Hq * D, probs, slse, dq + (size_t)r0 * Hq * D,
        dk + (size_t)r0 * Hkv * D, dv + (size_t)r0 * Hkv * D, L, Hq, Hkv, D,
        freq_base);
    for (int h = 0; h < Hq; h++)
      memcpy(lse + (size_t)h * T + r0, slse + (size_t)h * L, sizeof(float) * L);
    free(probs);
    free(slse);
    if (rc) return rc;
  }
  return 0;
}

/* Seeded inputs shared by tests and bench: SplitMix64 -> Box-Muller fp32,
 * value = mean + std * z.  Deterministic on every platform. */
static uint64_t splitmix64(uint64_t *s) {
  uint64_t z = (*s += 0x9E3779B97F4A7C15ull);
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

void oracle_fill_normal(float *x, size_t n, uint64_t seed, float mean,
                        float std) {
  uint64_t s = seed;
  for (size_t i = 0; i < n; i += 2) {
    double u1 = ((double)(splitmix64(&s) >> 11) + 1.0) * (1.0 / 9007199254740992.0);
    double u2 = (double)(splitmix64(&s) >> 11) * (1.0 / 9007199254740992.0);
    double r = sqrt(-2.0 * log(u1));
    double a = 6.283185307179586 * u2;
    x[i] = (float)(mean + std * r * cos(a));
    if (i + 1 < n) x[i + 1] = (float)(mean + std * r * sin(a));
  }
}

int oracle_num_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

void oracle_set_num_threads(int n) {
#ifdef _OPENMP
  if (n > 0) omp_set_num_threads(n);
#else
  (void)n;
#endif
}
