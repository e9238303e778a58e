/*
 * sophia_kda.h -- C ABI of the MI355X (gfx950) Kimi Delta Attention hot path.
 *
 * Plain pointers and sizes only: every tensor argument is a device pointer
 * into HBM, every size is an element count, and `stream` is a hipStream_t
 * passed as void* (NULL = the default stream).  Calls are asynchronous on
 * `stream`; no call allocates device memory or synchronises the device.
 *
 * Each entry point returns SOPHIA_OK (0) or an error code; the message of the
 * last failure on the calling thread is returned by sophia_last_error().
 * Shape / dtype / pointer errors are detected on the host before any launch.
 *
 * Reference interfaces replaced (Arain119/Sophia):
 *   sophia_short_conv_fwd   CausalDepthwiseConv1d.forward
 *                           (ml/runtime/model/attention.py:32-60) as driven by
 *                           SophiaKDA._short_convolution (attention.py:226-258),
 *                           and causal_conv1d_fn
 *                           (ml/training/pretrain/engine/sm120_concurrent_ffn.py:199-207)
 *   sophia_short_conv_step  the same forward with T == 1 and the cached
 *                           history conv_state[:B] (attention.py:236-237,251-257)
 *   sophia_kda_chunk_fwd    fla.ops.kda.chunk_kda as called at attention.py:349-365
 *                           with the varlen contract of FlashKDA
 *                           (sm120_concurrent_ffn.py:209-268,375-423: cu_seqlens,
 *                           chunk_size = 64, safe_gate, lower_bound, A_log, dt_bias)
 *   sophia_kda_decode_step  fla.ops.kda.fused_recurrent_kda as called at
 *                           attention.py:330-348 (T == 1 with a cached state)
 *   sophia_kda_decode_conv_step  the two above in one launch (the conv step of
 *                           attention.py:236-257 followed by 330-348)
 *   sophia_kda_conv_chunk_fwd  sophia_short_conv_fwd over the q, k, v channels
 *                           followed by sophia_kda_chunk_fwd, the conv inside the
 *                           prefill's intra-chunk kernel (the prefill rows of
 *                           SophiaKDA.forward: attention.py:226-258 then 349-365)
 *   sophia_kda_chunk_bwd    FlashKDA's chunk_kda_train_bwd with l2norm_bwd and
 *                           fused_beta_sigmoid_bwd, as FlashKDAFunction.backward
 *                           calls them (sm120_concurrent_ffn.py:301-373)
 */
#ifndef SOPHIA_KDA_H
#define SOPHIA_KDA_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes -------------------------------------------------------- */
#define SOPHIA_OK 0
#define SOPHIA_ERR_INVALID 1   /* bad shape, dtype, size or NULL pointer      */
#define SOPHIA_ERR_HIP 2       /* HIP runtime reported an error on launch      */
#define SOPHIA_ERR_WORKSPACE 3 /* workspace smaller than the size query says  */

/* ---- element types ------------------------------------------------------- */
#define SOPHIA_DTYPE_F32 0
#define SOPHIA_DTYPE_BF16 1

/* ---- KDA core switches (the use_*_in_kernel flags of chunk_kda) ---------- */
#define SOPHIA_KDA_QK_L2NORM 1u      /* q,k <- q/|q|, k/|k| (eps 1e-12)        */
#define SOPHIA_KDA_GATE_IN_KERNEL 2u /* g <- lb*sigmoid(exp(A_log[h])*(g+dt_bias)) */
#define SOPHIA_KDA_BETA_SIGMOID 4u   /* beta <- sigmoid(beta)                   */
/* Prefill launch switch: keep one scan chain per sequence.  Without it, a
 * batch of at most 4 sequences with host offsets whose longest sequence has
 * at least 128 chunks is scanned segment-parallel (its results then differ
 * from the single chain by rounding only). */
#define SOPHIA_KDA_SCAN_NO_SEGMENTS 8u
/* Backward switch (sophia_kda_chunk_bwd): the per-token recurrent form in
 * fp32 arithmetic instead of the chunk form on bf16 MFMA operands (fp32
 * accumulation and state, the forward's arithmetic). */
#define SOPHIA_KDA_BWD_RECURRENT 16u
/* Backward switch (sophia_kda_chunk_bwd): dq, dk and dv are written as bf16
 * (each the fp32 gradient rounded to nearest even), the element type a bf16
 * forward's q, k, v carry; dg, dbeta and the state gradients stay fp32. */
#define SOPHIA_KDA_BWD_GRAD_BF16 32u

/* Message of the last failing call on this thread ("" if none). */
const char *sophia_last_error(void);

/* ABI version of this library (major * 100 + minor). */
int sophia_abi_version(void);

/*
 * Depthwise causal conv (kernel K, SiLU) over a packed ragged batch.
 *   x, y        : [total_tokens, channels] rows; row strides in elements.
 *                 dtype SOPHIA_DTYPE_F32 or _BF16 (same for x and y).
 *   weight      : [channels, K] fp32, weight[:, K-1] multiplies the newest token.
 *   cu_seqlens  : [n_seqs + 1] int32 device offsets, cu_seqlens[0] == 0,
 *                 cu_seqlens[n_seqs] == total_tokens.
 *   conv_state  : [n_state_slots, channels, K-1] fp32 or NULL.  Sequence s uses
 *                 slot state_slots[s] (or s when state_slots is NULL); a slot
 *                 outside [0, n_state_slots) means no history: zeros are read
 *                 and nothing is written.
 *   read_history: 1 = the K-1 samples before each sequence come from
 *                 conv_state, 0 = zeros.
 *   write_history: 1 = conv_state[slot] <- last K-1 samples of cat(history, x).
 * y[t, c] = silu(sum_j weight[c, j] * seq[t + j]), seq = cat(history, x).
 */
int sophia_short_conv_fwd(const void *x, int64_t x_row_stride, void *y, int64_t y_row_stride,
                          int dtype, const float *weight, float *conv_state, int n_state_slots,
                          const int32_t *state_slots, const int32_t *cu_seqlens, int n_seqs,
                          int64_t total_tokens, int channels, int kernel_size, int read_history,
                          int write_history, void *stream);

/*
 * One-token conv step for `batch` sequences (decode).  x, y: [batch, channels]
 * rows; conv_state / slots as above, read when read_history != 0 and always
 * updated (rows whose slot is out of range run with zero history, no update).
 */
int sophia_short_conv_step(const void *x, int64_t x_row_stride, void *y, int64_t y_row_stride,
                           int dtype, const float *weight, float *conv_state, int n_state_slots,
                           const int32_t *state_slots, int batch, int channels, int kernel_size,
                           int read_history, void *stream);

/*
 * Backward of sophia_short_conv_fwd (training): the gradients of x and of the
 * taps for an output gradient dy.  Replaces the backward of causal_conv1d_fn
 * that the reference's training plugin installs as the conv forward
 * (ml/training/pretrain/engine/sm120_concurrent_ffn.py:199-207,425-428), and
 * autograd through CausalDepthwiseConv1d.forward (attention.py:32-60).
 *   x, weight, conv_state, state_slots, cu_seqlens, read_history: as in the
 *                 forward call (the history it read; the history itself gets
 *                 no gradient).  weight: the taps the forward used, fp32 [C, K].
 *   dy          : [total_tokens, channels] gradient of y, dtype `dtype` (x's).
 *   dx          : [total_tokens, channels] out, dtype `dtype`; rows outside
 *                 every sequence get zeros.
 *   dweight     : [channels, K] fp32 out, summed over all tokens in a fixed
 *                 order (deterministic).
 *   x, dy, dx   : 4-element aligned rows, strides multiples of 4 elements.
 * workspace: device memory of sophia_short_conv_bwd_workspace_size() bytes.
 */
size_t sophia_short_conv_bwd_workspace_size(int64_t total_tokens, int channels, int kernel_size);
int sophia_short_conv_bwd(const void *x, int64_t x_row_stride, const void *dy, int64_t dy_row_stride,
                          void *dx, int64_t dx_row_stride, int dtype, const float *weight,
                          const float *conv_state, int n_state_slots, const int32_t *state_slots,
                          const int32_t *cu_seqlens, int n_seqs, int64_t total_tokens, int channels,
                          int kernel_size, int read_history, float *dweight, void *workspace,
                          size_t workspace_bytes, void *stream);

/*
 * Workspace bytes needed by sophia_kda_chunk_fwd for a packed batch of
 * `total_tokens` tokens in `n_seqs` sequences with `num_heads` heads
 * (head_dim 128).  Depends only on these sizes, never on the offsets.
 */
size_t sophia_kda_chunk_workspace_size(int64_t total_tokens, int n_seqs, int num_heads,
                                       int head_dim);

/*
 * Chunkwise (C = 64) gated delta-rule prefill over a packed ragged batch.
 *   q, k        : [total_tokens, H, 128] rows of stride qkv_row_stride elements
 *                 (head h at element offset h*128 inside a row); dtype qkv_dtype.
 *   v           : same layout as q, value dim 128.
 *   g           : [total_tokens, H, 128], row stride g_row_stride, dtype g_dtype;
 *                 decay logits when SOPHIA_KDA_GATE_IN_KERNEL is set, else the
 *                 log-decay itself.  The log-decay must lie in [lower_bound, 0]
 *                 with lower_bound >= -5 (the safe-gate range of the kernel).
 *   beta        : [total_tokens, H], row stride beta_row_stride, dtype beta_dtype.
 *   A_log, dt_bias: [H] and [H*128] fp32 (read only with GATE_IN_KERNEL).
 *   scale       : multiplier of q (chunk_kda default 128^-0.5).
 *   initial_state, final_state: [n_state_slots, H, 128, 128] fp32 (state[k][v])
 *                 or NULL (zero initial state / final state not written);
 *                 sequence s uses slot state_slots[s] (or s); they may alias.
 *                 A slot outside [0, n_state_slots) starts from zero and is
 *                 not written.
 *   o           : [total_tokens, H, 128] rows of stride o_row_stride, dtype qkv_dtype.
 *   cu_seqlens_host: NULL, or a host copy of cu_seqlens (FlashKDA's
 *                 cu_seqlens_cpu, sm120_concurrent_ffn.py:231).  It shapes
 *                 the launch (longest sequences first, more work-groups per
 *                 chain for long chains, segments for a few long sequences --
 *                 see SOPHIA_KDA_SCAN_NO_SEGMENTS); results are identical with
 *                 or without it, but for the rounding of segmented chains.
 *                 Must be non-decreasing within [0, total_tokens].
 *   workspace   : device scratch of sophia_kda_chunk_workspace_size() bytes,
 *                 256-byte aligned; contents need not be initialised.
 */
int sophia_kda_chunk_fwd(const void *q, const void *k, const void *v, int64_t qkv_row_stride,
                         int qkv_dtype, const void *g, int64_t g_row_stride, int g_dtype,
                         const void *beta, int64_t beta_row_stride, int beta_dtype,
                         const float *A_log, const float *dt_bias, float scale, float lower_bound,
                         unsigned flags, const int32_t *cu_seqlens,
                         const int32_t *cu_seqlens_host, int n_seqs,
                         int64_t total_tokens, int num_heads, int head_dim,
                         const float *initial_state, float *final_state, int n_state_slots,
                         const int32_t *state_slots, void *o, int64_t o_row_stride,
                         void *workspace, size_t workspace_bytes, void *stream);

/*
 * sophia_kda_chunk_fwd without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  No counterpart in the reference: it
 * exists for those callers only.  Same arguments, kernels and results as
 * sophia_kda_chunk_fwd; the scratch is a static device array of
 * SOPHIA_KDA_CHUNK_NO_ALLOC_MAX_BYTES bytes inside this library (one per
 * device, held until the process ends), so a batch whose
 * sophia_kda_chunk_workspace_size() exceeds that returns
 * SOPHIA_ERR_WORKSPACE (16 heads: up to 903 (chunk, head) records, e.g. one
 * sequence of 3,520 tokens, or 24 sequences totalling 2,048 tokens).  All
 * calls on one device share that array: calls that overlap in time on one
 * device (several streams, several host threads) race and must be ordered
 * by the caller.  Allocates nothing and synchronises nothing.
 */
#define SOPHIA_KDA_CHUNK_NO_ALLOC_MAX_BYTES ((size_t)64 << 20)
int sophia_kda_chunk_fwd_no_alloc(const void *q, const void *k, const void *v,
                                  int64_t qkv_row_stride, int qkv_dtype, const void *g,
                                  int64_t g_row_stride, int g_dtype, const void *beta,
                                  int64_t beta_row_stride, int beta_dtype, const float *A_log,
                                  const float *dt_bias, float scale, float lower_bound,
                                  unsigned flags, const int32_t *cu_seqlens,
                                  const int32_t *cu_seqlens_host, int n_seqs,
                                  int64_t total_tokens, int num_heads, int head_dim,
                                  const float *initial_state, float *final_state,
                                  int n_state_slots, const int32_t *state_slots, void *o,
                                  int64_t o_row_stride, void *stream);

/*
 * One recurrent step for `batch` sequences, state updated in place.
 *   q, k, v, g : [batch, H, 128] rows (strides in elements), beta: [batch, H].
 *   state      : [n_state_slots, H, 128, 128] fp32; row b uses slot
 *                state_slots[b] (or b); an out-of-range slot leaves the state
 *                untouched and the row's output 0.  read_state == 0 treats
 *                the incoming state as zero.
 *   o          : [batch, H, 128] rows of stride o_row_stride, dtype qkv_dtype.
 */
int sophia_kda_decode_step(const void *q, const void *k, const void *v, int64_t qkv_row_stride,
                           int qkv_dtype, const void *g, int64_t g_row_stride, int g_dtype,
                           const void *beta, int64_t beta_row_stride, int beta_dtype,
                           const float *A_log, const float *dt_bias, float scale,
                           float lower_bound, unsigned flags, float *state, int n_state_slots,
                           const int32_t *state_slots, int read_state, int batch, int num_heads,
                           int head_dim, void *o, int64_t o_row_stride, void *stream);

/*
 * One decode step of a KDA layer with its ShortConv: the one-token conv of
 * the q, k and v channels (CausalDepthwiseConv1d.forward with T == 1 on the
 * cached history, attention.py:32-60,236-257) followed by the recurrent step
 * of sophia_kda_decode_step, in one launch.
 *   x_q, x_k, x_v : [batch, H, 128] pre-conv projection rows (row stride
 *                   x_row_stride elements, dtype qkv_dtype); the conv output is
 *                   rounded to that dtype, as the separate ShortConv writes it.
 *   conv_weight   : [3 * H * 128, kernel_size] fp32 taps (q | k | v channels,
 *                   rounded to the activation dtype), 16-byte aligned.
 *   conv_state    : [n_state_slots, 3 * H * 128, kernel_size - 1] fp32 history,
 *                   the slot of each row shifted by one token in place.
 *   kernel_size   : 4.
 * Other arguments as sophia_kda_decode_step; read_state == 0 treats both the
 * recurrent state and the conv history as zero.  Results are those of
 * sophia_short_conv_step followed by sophia_kda_decode_step.
 */
int sophia_kda_decode_conv_step(const void *x_q, const void *x_k, const void *x_v, int64_t x_row_stride,
                                int qkv_dtype, const float *conv_weight, float *conv_state, int kernel_size,
                                const void *g, int64_t g_row_stride, int g_dtype, const void *beta,
                                int64_t beta_row_stride, int beta_dtype, const float *A_log,
                                const float *dt_bias, float scale, float lower_bound, unsigned flags,
                                float *state, int n_state_slots, const int32_t *state_slots, int read_state,
                                int batch, int num_heads, int head_dim, void *o, int64_t o_row_stride,
                                void *stream);

/*
 * The prefill of a KDA layer with its ShortConv: the causal conv + SiLU of the
 * q, k and v channels over each sequence (CausalDepthwiseConv1d.forward,
 * attention.py:32-60, as SophiaKDA._short_convolution drives it, 226-258)
 * computed inside the chunk prefill's intra-chunk kernel from the rows before
 * the conv, then the prefill of sophia_kda_chunk_fwd (attention.py:349-365).
 * The conv outputs never reach memory.
 *   x_q, x_k, x_v : [total, H, 128] bf16 projection rows before the conv (row
 *                   stride x_row_stride elements, a multiple of 8; 16-byte
 *                   aligned); each conv output is rounded to bf16, as the
 *                   separate ShortConv writes it.
 *   conv_weight   : [3 * H * 128, kernel_size] fp32 taps (q | k | v channels),
 *                   16-byte aligned.
 *   conv_state    : [n_state_slots, 3 * H * 128, kernel_size - 1] fp32 histories
 *                   (16-byte aligned) or NULL: sequence s uses slot
 *                   state_slots[s] (or s), read when read_history != 0 (else,
 *                   and for a slot outside [0, n_state_slots), zeros) and
 *                   replaced by the last kernel_size - 1 rows of
 *                   cat(history, x) of the sequence.
 *   kernel_size   : 4.
 * Other arguments, the workspace size and the states as sophia_kda_chunk_fwd
 * (q, k, v being the conv outputs; n_seqs <= 65535).  Results are bitwise those
 * of sophia_short_conv_fwd (write_history = 1) followed by sophia_kda_chunk_fwd.
 */
int sophia_kda_conv_chunk_fwd(const void *x_q, const void *x_k, const void *x_v, int64_t x_row_stride,
                              int qkv_dtype, const float *conv_weight, float *conv_state, int kernel_size,
                              int read_history, const void *g, int64_t g_row_stride, int g_dtype,
                              const void *beta, int64_t beta_row_stride, int beta_dtype, const float *A_log,
                              const float *dt_bias, float scale, float lower_bound, unsigned flags,
                              const int32_t *cu_seqlens, const int32_t *cu_seqlens_host, int n_seqs,
                              int64_t total_tokens, int num_heads, int head_dim, const float *initial_state,
                              float *final_state, int n_state_slots, const int32_t *state_slots, void *o,
                              int64_t o_row_stride, void *workspace, size_t workspace_bytes, void *stream);

/*
 * Backward of the prefill (training).  Replaces FlashKDA's chunk_kda_train_bwd
 * followed by l2norm_bwd and fused_beta_sigmoid_bwd, as FlashKDAFunction.
 * backward calls them (ml/training/pretrain/engine/sm120_concurrent_ffn.py:
 * 301-373): the gradients of o = KDA(q, k, v, g, beta; h0) and of its final
 * states with respect to every input, the l2 norms, the gate and the beta
 * sigmoid included (same flags as sophia_kda_chunk_fwd).
 *   q, k, v, g, beta, A_log, dt_bias, scale, lower_bound, flags, cu_seqlens,
 *                     n_seqs, total_tokens, num_heads, head_dim:
 *                     the forward's inputs, as for sophia_kda_chunk_fwd.
 *   initial_state   : [n_seqs, H, 128, 128] fp32 per sequence, or NULL (zeros).
 *   d_out           : [total, H, 128] gradient of o (row stride in elements),
 *                     dtype SOPHIA_DTYPE_F32 or _BF16.
 *   d_final_state   : [n_seqs, H, 128, 128] fp32 gradient of the final states,
 *                     or NULL (zeros).
 * Outputs, fp32 (dq, dk, dv bf16 with SOPHIA_KDA_BWD_GRAD_BF16), dense:
 *   dq, dk, dv, dg  : [total, H, 128]   (dg with respect to the g input: the
 *                                        decay logits when the gate is applied
 *                                        in the kernel, else the log-decay)
 *   dbeta           : [total, H]         (with respect to the beta input)
 *   d_initial_state : [n_seqs, H, 128, 128] or NULL (not computed)
 *   dA_log          : [H] or NULL        (only with SOPHIA_KDA_GATE_IN_KERNEL)
 *   ddt_bias        : [H * 128] or NULL  (only with SOPHIA_KDA_GATE_IN_KERNEL)
 * Rows outside [cu_seqlens[0], cu_seqlens[n_seqs]) belong to no sequence: their
 * dq, dk, dv, dg, dbeta are zero and they add nothing to dA_log / ddt_bias.
 * workspace: device memory of sophia_kda_chunk_bwd_workspace_size() bytes,
 * 256-byte aligned.
 * Arithmetic.  The default chunk form follows the forward's chunk form: its
 * per-chunk operands (the forward's records, the states and state gradients
 * fed to the two chunk scans) are bf16 MFMA operands with fp32 accumulation
 * and fp32 states; the per-chunk gradient products split each fp32 operand
 * into two bf16 parts (hi + lo, ~16 mantissa bits) and sum hi*hi + hi*lo +
 * lo*hi in fp32.  Its error against an fp64 backward is that of the forward's
 * bf16 operands (measured 1.4e-3 to 8e-3 relative, max-norm).  With
 * SOPHIA_KDA_BWD_RECURRENT in flags the per-token recurrence runs in fp32
 * throughout (~1e-7 relative, several times slower).  Sums over tokens and
 * value columns run in a fixed order in both forms (results are deterministic).
 */
size_t sophia_kda_chunk_bwd_workspace_size(int64_t total_tokens, int n_seqs, int num_heads,
                                           int head_dim);
int sophia_kda_chunk_bwd(const void *q, const void *k, const void *v, int64_t qkv_row_stride,
                         int qkv_dtype, const void *g, int64_t g_row_stride, int g_dtype,
                         const void *beta, int64_t beta_row_stride, int beta_dtype, const float *A_log,
                         const float *dt_bias, float scale, float lower_bound, unsigned flags,
                         const int32_t *cu_seqlens, int n_seqs, int64_t total_tokens, int num_heads,
                         int head_dim, const float *initial_state, const void *d_out,
                         int64_t d_out_row_stride, int d_out_dtype, const float *d_final_state, void *dq,
                         void *dk, void *dv, float *dg, float *dbeta, float *d_initial_state,
                         float *dA_log, float *ddt_bias, void *workspace, size_t workspace_bytes,
                         void *stream);

#ifdef __cplusplus
}
#endif

#endif /* SOPHIA_KDA_H */
