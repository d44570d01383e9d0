/*
 * glacier_attn.h -- C ABI of libglacier_attn.so: MI355X (gfx950) causal
 * grouped-query self-attention, forward and backward, for Glacier.Tune.
 *
 * The path: RoPE on Q/K (NeoX half-split), QK^T with the causal mask, row
 * softmax, PV; and the reverse (dP, softmax gradient, dQ/dK/dV with the GQA
 * head reduction, inverse RoPE).  The forward saves the row log-sum-exp
 * instead of the [Hq,S,S] probability matrix; the backward recomputes P from
 * it.  Calling the forward again with an lse buffer is the activation-
 * checkpoint recompute; it is bitwise identical to the first call.
 *
 * Layouts (all row-major, token-major, heads interleaved, exactly the C#
 * tensors of TransformerBlock, CausalAttentionKernel.cs:33,40):
 *   q, attn_out, d_attn_out, dq : [T][Hq][D]
 *   k, v, dk, dv                : [T][Hkv][D]
 *   lse                         : [Hq][T] fp32, natural log of
 *                                 sum_{j<=i} exp(q_i.k_j / sqrt(D))
 * where T is the token count (S for one sequence) and query head h reads KV
 * head h / (Hq/Hkv).
 *
 * Every entry point returns a GLACIER_ATTN_* status; on failure the text is
 * in glacier_attn_last_error() (per calling thread).  All arguments are
 * validated before the GPU is touched.  One call at a time per context (the
 * library also serialises calls on a context with a mutex, as
 * GpuLoraEngine._scratchLock does).  The caller owns every tensor; the
 * library writes only to the outputs named below and owns only its scratch.
 */
#ifndef GLACIER_ATTN_H
#define GLACIER_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ------------------------------------------------------ */
#define GLACIER_ATTN_OK 0
/* a bad argument (null pointer, Hq % Hkv != 0, non-positive size ...);
 * GpuLoraEngine throws ArgumentOutOfRangeException for these
 * (GpuLoraEngine.Forward.cs:437-438) */
#define GLACIER_ATTN_ERR_INVALID_ARGUMENT 1
/* valid, but outside what the GPU kernels cover (head_dim other than 32, 64,
 * 96, 128 or 256; 256 in GLACIER_ATTN_PREC_FP32; a sequence longer than
 * GLACIER_ATTN_MAX_SEQ_LEN): the caller keeps its CPU path, like the
 * canUseGpuAttn gate (TransformerBlock.cs:428-434) */
#define GLACIER_ATTN_ERR_UNSUPPORTED 2
/* a HIP runtime or launch failure (CuDriver.Check, GpuLoraEngine.Forward.cs:457-464) */
#define GLACIER_ATTN_ERR_DEVICE 3
/* device memory could not be allocated */
#define GLACIER_ATTN_ERR_OUT_OF_MEMORY 4

/* ---- precision and device-buffer dtypes --------------------------------- */
/* fp32 operands, fp32 MFMA (the correctness mode) */
#define GLACIER_ATTN_PREC_FP32 0
/* bf16 operands on the matrix cores, fp32 accumulation, fp32 softmax
 * statistics; q/k rotated in fp32 before rounding to bf16 */
#define GLACIER_ATTN_PREC_BF16 1

#define GLACIER_ATTN_IO_F32 0  /* device tensors are float */
#define GLACIER_ATTN_IO_BF16 1 /* device tensors are bfloat16 (PREC_BF16 only) */

/* longest single sequence the kernels take (keys of one sequence) */
#define GLACIER_ATTN_MAX_SEQ_LEN 65536

typedef struct glacier_attn_ctx glacier_attn_ctx;

/* Shape of one call on device-resident tensors. */
typedef struct glacier_attn_desc {
  int32_t total_tokens;       /* T: rows of q/k/v (sum of the sequence lengths) */
  int32_t n_seqs;             /* 1, or the number of packed sequences */
  const int32_t *cu_seqlens;  /* host array of n_seqs+1 token offsets
                                 (0 = cu[0] <= ... <= cu[n] = T), or NULL for
                                 one sequence of T tokens.  Sequences do not
                                 attend to each other; RoPE positions restart
                                 at 0 in each. */
  int32_t n_heads_q;
  int32_t n_heads_kv;
  int32_t head_dim;
  float rope_freq_base;       /* theta; 1/theta^(2i/D) per pair (RoPEKernel.cs:64) */
  int32_t precision;          /* GLACIER_ATTN_PREC_* */
  int32_t io_dtype;           /* GLACIER_ATTN_IO_* of every device tensor except lse */
} glacier_attn_desc;

/* ---- context ------------------------------------------------------------ */

/* Creates a context on HIP device `device_ordinal` with its own stream and
 * grow-only scratch; `precision` is what the *_host entry points use.
 * Replaces the attention part of the GpuLoraEngine constructor
 * (GpuLoraEngine.cs:114-155 function loads, :205-208 attention scratch).
 * If it fails the caller keeps its CPU path (GgufLoraModel.cs:66-80). */
int glacier_attn_create(int device_ordinal, int precision, glacier_attn_ctx **out);

/* Frees the context and everything it owns (GpuLoraEngine.Dispose). */
void glacier_attn_destroy(glacier_attn_ctx *ctx);

/* Text of the last failure on the calling thread ("" if none). */
const char *glacier_attn_last_error(void);

/* 1 if the GPU kernels take this shape, else 0: 1 <= head_dim <= 256 and
 * 1 <= seq_len <= GLACIER_ATTN_MAX_SEQ_LEN.  The kernels are built for head
 * sizes 32, 64, 96, 128 and 256; any other size runs them on rows padded to
 * the next of those (with the RoPE pairs kept, so results are those of the
 * call's own size).  Sizes padded to 256 run in GLACIER_ATTN_PREC_BF16 only
 * (fp32 key/value tiles of 256 exceed the LDS), and the allocation-free
 * backward takes the built sizes only.  Replaces
 * GpuLoraEngine.SupportsAttention (GpuLoraEngine.cs:111-112), which accepts
 * head_dim 1..1024; sizes above 256 keep the CPU path. */
int glacier_attn_supports(int seq_len, int head_dim);

/* ---- drop-in entry points: host fp32 tensors ----------------------------- */

/* GpuLoraEngine.ForwardAttention (GpuLoraEngine.Forward.cs:467-512): q, k,
 * v are the pre-RoPE projections [S][H][D].  attn_out is overwritten.  When
 * attn_lse is not NULL (the state is being saved: the reference passes a
 * probs tensor there) q and k are overwritten with their post-RoPE values
 * (GpuLoraEngine.Forward.cs:496-500) and attn_lse [Hq][S] receives the row
 * log-sum-exp that BackwardAttention needs in place of probs.  When it is
 * NULL (inference, or the first pass under activation checkpointing) q and
 * k are left untouched.  layer_index is accepted for signature parity and
 * not used, as in the reference. */
int glacier_attn_forward_host(glacier_attn_ctx *ctx, int layer_index, float *q,
                              float *k, const float *v, float *attn_out,
                              float *attn_lse, int seq_len, int n_heads_q,
                              int n_heads_kv, int head_dim,
                              float rope_freq_base);

/* GpuLoraEngine.BackwardAttention (GpuLoraEngine.Backward.cs:414-458): q,
 * k are the post-RoPE values saved by the forward, v as saved, d_attn_out
 * the upstream gradient, attn_out the saved forward output (the reference's
 * state.AttnOut, TransformerBlock.cs:496; it gives the softmax-gradient row
 * term D_i = dO_i . O_i), attn_lse the saved log-sum-exp.  dq and dk are
 * gradients w.r.t. the pre-RoPE inputs (inverse rotation applied,
 * GpuLoraEngine.Backward.cs:452); dv plain.  dq, dk, dv are overwritten, not
 * accumulated (CausalAttentionKernel.cs:90-92). */
int glacier_attn_backward_host(glacier_attn_ctx *ctx, int layer_index,
                               const float *d_attn_out, const float *q,
                               const float *k, const float *v,
                               const float *attn_out, const float *attn_lse,
                               float *dq, float *dk, float *dv, int seq_len,
                               int n_heads_q, int n_heads_kv, int head_dim,
                               float rope_freq_base);

/* ---- device entry points: tensors already in HBM ------------------------- */

/* LaunchRopeBatch + LaunchAttnTrainFwd (GpuLoraEngine.Forward.cs:401-465)
 * on device pointers, enqueued on the context's stream (asynchronous).
 * q, k, v: pre-RoPE inputs.  out: attention output.  lse: [Hq][T] fp32 or
 * NULL.  q_rot, k_rot: receive the post-RoPE q/k (same layout and dtype as
 * q/k) or NULL.  Outputs must not alias inputs. */
int glacier_attn_forward(glacier_attn_ctx *ctx, const glacier_attn_desc *desc,
                         const void *q, const void *k, const void *v, void *out,
                         float *lse, void *q_rot, void *k_rot);

/* LaunchAttnTrainBwd + inverse LaunchRopeBatch (GpuLoraEngine.Backward.cs:354-412,
 * :452) on device pointers, enqueued on the context's stream.  d_out: dO;
 * q_rot, k_rot: post-RoPE q/k from the forward; out, lse: forward output and
 * log-sum-exp.  dq, dk: gradients w.r.t. pre-RoPE q/k; dv. */
int glacier_attn_backward(glacier_attn_ctx *ctx, const glacier_attn_desc *desc,
                          const void *d_out, const void *q_rot,
                          const void *k_rot, const void *v, const void *out,
                          const float *lse, void *dq, void *dk, void *dv);

/* ---- allocation-free backward ------------------------------------------- */

/* Bytes of the fixed device array behind glacier_attn_backward_noalloc: 80
 * MiB, held by every GPU that loads the library until the process ends. */
#define GLACIER_ATTN_NOALLOC_SCRATCH_BYTES (80u * 1024u * 1024u)

/* glacier_attn_backward without any device allocation.  It has no
 * counterpart in the reference: it is for callers that cannot allocate
 * (code recorded under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc).  Same arguments, kernels and results (bitwise) as
 * glacier_attn_backward, and it calls no hipMalloc, hipFree or other
 * allocating routine; every buffer beyond the caller's tensors lives in one
 * fixed device array of GLACIER_ATTN_NOALLOC_SCRATCH_BYTES per GPU, laid
 * out per call as (each part rounded up to 256 bytes)
 *   RoPE cos and sin tables    2 x 4 * ceil_256(L) * D/2   (L: longest sequence)
 *   tile and position tables   32 * tiles + 32 * wtiles + 4 * T
 *                              (tiles: sum of ceil(len/64); wtiles: sum of
 *                              ceil(len/128) for bf16 tensors at head_dim 64
 *                              or 128, else 0; 48 * wtiles when the wide
 *                              backward takes query heads in pairs)
 *   row stats (bf16 tensors)   8 * (T * Hq + 64)
 *   dK and dV partials         2 x esz * T * Hq * D        (esz 2 bf16, 4 fp32 tensors)
 * A call that needs more, or has more than 1024 sequences or 65536 tokens,
 * returns GLACIER_ATTN_ERR_UNSUPPORTED and leaves the outputs untouched.
 * The first call with a new sequence layout, head_dim, theta or a longer
 * sequence than the array's tables cover waits for the whole device and
 * uploads the tables (synchronous copies: make that call before capturing
 * a graph); calls that repeat a layout only enqueue the kernels.  The array
 * is shared by every call on the GPU, from any context, stream or thread,
 * and keeps the last call's contents: calls that overlap on one GPU race,
 * so the caller serialises them. */
int glacier_attn_backward_noalloc(glacier_attn_ctx *ctx, const glacier_attn_desc *desc,
                                  const void *d_out, const void *q_rot,
                                  const void *k_rot, const void *v, const void *out,
                                  const float *lse, void *dq, void *dk, void *dv);

/* Makes every entry point enqueue on `hip_stream` (a hipStream_t; NULL is
 * the HIP null stream).  A new context uses a non-blocking stream of its own
 * (default priority). */
int glacier_attn_set_stream(glacier_attn_ctx *ctx, void *hip_stream);

/* Returns the context to its own stream. */
int glacier_attn_use_own_stream(glacier_attn_ctx *ctx);

/* Waits for everything enqueued by this context. */
int glacier_attn_synchronize(glacier_attn_ctx *ctx);

/* ---- instrumentation (no reference counterpart: the reference times its
 * phases with Stopwatch, TransformerBlock.cs:311-321) ---------------------- */

/* Enables (1) or disables (0) per-kernel hipEvent timing on the context's
 * stream; enabling clears the counters. */
int glacier_attn_set_kernel_timing(glacier_attn_ctx *ctx, int enable);

/* Number of kernel kinds the library launches. */
int glacier_attn_kernel_count(void);

/* Name of kernel kind `id`, or NULL. */
const char *glacier_attn_kernel_name(int id);

/* Summed device time (ms) and launch count of kernel kind `id` since timing
 * was enabled; synchronises the context's stream. */
int glacier_attn_kernel_time(glacier_attn_ctx *ctx, int id, double *total_ms,
                             int64_t *launches);

#ifdef __cplusplus
}
#endif

#endif /* GLACIER_ATTN_H */
