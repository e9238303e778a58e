/*
 * sophia_decoder.h -- C ABI of the decoder-side kernels of the MI355X build:
 * the layers between the KDA mixers of the hybrid decoder.
 *
 * Conventions as in sophia_kda.h: device pointers, strides in elements, an
 * explicit hipStream_t passed as void*, an int status (SOPHIA_OK or an error
 * code; sophia_last_error() describes the last failure).  Nothing here
 * allocates or synchronises.  dtype is SOPHIA_DTYPE_F32 or SOPHIA_DTYPE_BF16
 * for every activation tensor; weights are fp32.
 */
#ifndef SOPHIA_DECODER_H
#define SOPHIA_DECODER_H

#include <stddef.h>
#include <stdint.h>

#include "sophia_kda.h"

#ifdef __cplusplus
extern "C" {
#endif

/*
 * Depth mixing of the attention-residual blocks; replaces
 * AttentionResidualMixer.forward (ml/runtime/model/blocks.py:38-48), and, when
 * out_norm_weight is not NULL, also the RMSNorm that consumes its output
 * (SophiaBlock's attn_norm / ffn_norm, blocks.py:72-87, and the final norm
 * of the logits path, ml/runtime/model/transformer.py:189,210 and
 * ml/runtime/model/ops.py:67-77):
 *   partial  <- partial + residual, written to partial_out, when residual is not NULL
 *              (the residual add SophiaBlock does before the mix, blocks.py:78-86)
 *   values = [completed[:, 0], ..., completed[:, n_blocks-1], partial]
 *   score_b = RMSNorm(values_b; norm_weight, eps) . query_weight
 *   mix = sum_b softmax_b(score) * values_b
 *   out = mix, or RMSNorm(mix; out_norm_weight, out_eps)
 *   partial   : [rows, dim], row stride partial_stride.
 *   residual, partial_out : [rows, dim] or NULL (both or neither), row strides
 *               residual_stride, partial_out_stride; partial_out may not alias
 *               partial, residual or out.
 *   completed : [rows, n_blocks, dim] with strides (completed_row_stride,
 *               completed_block_stride, 1); unused when n_blocks == 0.
 *   norm_weight, query_weight, out_norm_weight : [dim] fp32.
 *   out       : [rows, dim], row stride out_stride (may not alias the inputs).
 * Sums, scores, softmax and the output norm run in fp32; out is rounded once.
 * dim a multiple of 8 and at most 4096; 0 <= n_blocks < 16; strides multiples
 * of 8; every pointer 16-byte aligned.
 */
int sophia_attn_res_mix(const void *partial, int64_t partial_stride, const void *residual, int64_t residual_stride,
                        void *partial_out, int64_t partial_out_stride, const void *completed,
                        int64_t completed_row_stride, int64_t completed_block_stride, int n_blocks,
                        const float *norm_weight, const float *query_weight, float eps,
                        const float *out_norm_weight, float out_eps, void *out, int64_t out_stride,
                        int64_t rows, int dim, int dtype, void *stream);

/*
 * SiTU-GLU hidden of FeedForward.forward (ml/runtime/model/blocks.py:23-27):
 *   g, u = gate_up[:, :hidden], gate_up[:, hidden:]
 *   out = gate_softcap tanh(g / gate_softcap) sigmoid(g) * up_softcap tanh(u / up_softcap)
 *   gate_up : [rows, 2 * hidden], row stride gate_up_stride.
 *   out     : [rows, hidden], row stride out_stride.
 * Computed in fp32, rounded once.  hidden a multiple of 8; strides multiples
 * of 8; pointers 16-byte aligned.
 */
int sophia_situ_glu(const void *gate_up, int64_t gate_up_stride, void *out, int64_t out_stride, int64_t rows,
                    int hidden, float gate_softcap, float up_softcap, int dtype, void *stream);

/*
 * Gated per-head output of the token mixers; replaces
 *   KDA: output_norm(o.to(dtype)) * sigmoid(gate)   (ml/runtime/model/attention.py:411-420)
 *   MLA: (o.float() * sigmoid(gate).float()).to(dtype)   (attention.py:655-656)
 * with norm_weight [head_dim] fp32 for the first form and NULL for the second:
 *   out[r, h, :] = (RMSNorm(o[r, h, :]; norm_weight, eps) or o[r, h, :]) * sigmoid(gate[r, h, :])
 *   o    : [rows, heads * head_dim], row stride o_stride, dtype o_dtype (fp32 or
 *          dtype; an fp32 o is rounded to dtype first, as the reference casts it).
 *   gate : [rows, heads * head_dim] logits, row stride gate_stride, dtype.
 *   out  : [rows, heads * head_dim], row stride out_stride, dtype.
 * head_dim a power of two in [8, 512]; strides multiples of 8; pointers
 * 16-byte aligned.  Computed in fp32, rounded once.
 */
int sophia_gated_head_norm(const void *o, int64_t o_stride, int o_dtype, const void *gate, int64_t gate_stride,
                           const float *norm_weight, float eps, void *out, int64_t out_stride, int64_t rows,
                           int heads, int head_dim, int dtype, void *stream);

/*
 * The normalisations after MLA's down projections (ml/runtime/model/
 * attention.py:611-614: q_norm(q_down(x)) and kv_norm(kv_down(x))) in place,
 * and each normalised latent row written into its latent-cache slot (the
 * cache write of attention.py:615-621, as the packed step places rows):
 *   q_lat  : [rows, q_rank], row stride q_stride; q_lat <- RMSNorm(q_lat; q_norm_weight, q_eps)
 *   kv_lat : [rows, kv_rank], row stride kv_stride; kv_lat <- RMSNorm(kv_lat; kv_norm_weight, kv_eps)
 *   dtype of both; the fp32 norm weights are rounded to it first, each output
 *   rounded once.  q_rank, kv_rank multiples of 8, q_rank + kv_rank <= 512.
 *   latent_cache : [n_slots, max_len, kv_rank] fp32, or NULL (no cache write).
 *     Prefill rows [0, n_prefill_rows): row i goes to
 *     (prefill_seq_slots[i / prefill_seq_len], i % prefill_seq_len) when
 *     prefill_seq_slots is given (equal-length prompts from position 0; it
 *     holds ceil(n_prefill_rows / prefill_seq_len) entries), else
 *     to (prefill_row_slots[i], prefill_row_pos[i]); decode row
 *     n_prefill_rows + j goes to (decode_slots[j], decode_pos[j]).  A slot or
 *     position out of range writes nothing.
 * Strides multiples of 8; pointers 16-byte aligned.
 */
int sophia_mla_latent_norms(void *q_lat, int64_t q_stride, void *kv_lat, int64_t kv_stride, int64_t rows,
                            int q_rank, int kv_rank, int dtype, const float *q_norm_weight, float q_eps,
                            const float *kv_norm_weight, float kv_eps, float *latent_cache, int n_slots,
                            int max_len, int64_t n_prefill_rows, const int32_t *prefill_seq_slots,
                            int prefill_seq_len, const int64_t *prefill_row_slots, const int64_t *prefill_row_pos,
                            const int32_t *decode_slots, const int64_t *decode_pos, void *stream);

/*
 * Backward of sophia_gated_head_norm (training): autograd through
 * output_norm(o) * sigmoid(output_gate(x)) (attention.py:411-420) and MLA's
 * o * sigmoid(gate) (attention.py:655-656).  d_out: [rows, heads * head_dim]
 * gradient of out (dtype); o, gate, norm_weight, eps, dtypes and strides as in
 * the forward call.  Outputs: d_o (o_dtype, the gradient of o before its
 * rounding to dtype), d_gate (dtype), and with norm_weight d_norm_weight
 * [head_dim] fp32, summed over rows and heads in a fixed order
 * (deterministic).  workspace: sophia_gated_head_norm_bwd_workspace_size()
 * bytes (used only with norm_weight).  head_dim a power of two in [8, 256].
 */
size_t sophia_gated_head_norm_bwd_workspace_size(int64_t rows, int heads, int head_dim);
int sophia_gated_head_norm_bwd(const void *d_out, int64_t d_out_stride, const void *o, int64_t o_stride,
                               int o_dtype, const void *gate, int64_t gate_stride, const float *norm_weight,
                               float eps, void *d_o, int64_t d_o_stride, void *d_gate, int64_t d_gate_stride,
                               float *d_norm_weight, int64_t rows, int heads, int head_dim, int dtype,
                               void *workspace, size_t workspace_bytes, void *stream);

/*
 * Absorbed MLA decode attention over the fp32 latent cache; replaces the
 * decode-row attention of SophiaMLA with NoPE (ml/runtime/model/attention.py:
 * 609-657 with a cache, keys = k_up(c), values = v_up(c)), written in latent
 * space: for each decode row b and head h, with qa[b, h] = W_k,h^T q[b, h],
 *   p = softmax_k(scale * qa[b, h] . latent[slot_b, k]),  k = 0 .. pos_b
 *   out[b, h] = sum_k p_k latent[slot_b, k]      (W_v,h is applied by the caller)
 *   qa      : [rows, heads, rank], row stride qa_stride (bf16 or fp32).
 *   latent  : [n_slots, max_seq, rank] fp32, slot stride slot_stride, rows of rank.
 *   slots   : [rows] int32; pos : [rows] int64 (keys 0..pos, clamped to max_seq;
 *             a row whose slot is outside [0, n_slots) gets zeros).
 *   out     : [rows, heads, rank], row stride out_stride (bf16 or fp32).
 * qa and the latents are rounded to bf16 for the products (the reference
 * casts both to the activation dtype); scores, softmax and sums are fp32.
 * rank in {32, 64, 128, 256}; heads <= 16.  splits > 1 divides each row's keys
 * among that many work-groups and needs a workspace of
 * sophia_mla_decode_workspace_size(rows, rank, splits) bytes.
 */
size_t sophia_mla_decode_workspace_size(int64_t rows, int rank, int splits);
int sophia_mla_decode_attn(const void *qa, int64_t qa_stride, int qa_dtype, const float *latent, int64_t slot_stride,
                           int n_slots, int max_seq, const int32_t *slots, const int64_t *pos, float scale, void *out,
                           int64_t out_stride, int out_dtype, int64_t rows, int heads, int rank, int splits,
                           void *workspace, size_t workspace_bytes, void *stream);

/*
 * Causal self-attention over packed sequences, bf16, head_dim 128; replaces
 * the prefill attention of SophiaMLA (ml/runtime/model/attention.py:630-654:
 * scaled_dot_product_attention with is_causal=True, or with the
 * tril(klen - seqlen) mask when the queries follow cached keys):
 *   out[t, h] = sum_{s <= t + off} softmax_s(scale * q[t, h] . k[s, h]) v[s, h]
 * over the query rows t of one sequence (cu_seqlens [n_seqs + 1] int32 on the
 * device) and its key/value rows s (cu_seqlens_k, or the same rows when
 * cu_seqlens_k is NULL), where off = keys - queries of that sequence: the
 * queries are the last positions of the key range (off = 0 for a prefill from
 * an empty cache).  total / total_k: rows of q / of k and v.  q, k, v, out:
 * [rows, heads, 128] with row strides in elements (q, k, v 16-byte aligned
 * with strides multiples of 8; out 8-byte aligned).  max_len must bound every
 * sequence's query count (it sizes the grid).  Scores, softmax and sums are
 * fp32; the probabilities enter the value product as bf16 (as they do in a
 * bf16 SDPA).
 */
int sophia_causal_attention(const void *q, int64_t q_stride, const void *k, int64_t k_stride, const void *v,
                            int64_t v_stride, void *out, int64_t out_stride, const int32_t *cu_seqlens,
                            const int32_t *cu_seqlens_k, int n_seqs, int64_t total, int64_t total_k, int max_len,
                            int heads, int head_dim, float scale, int dtype, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* SOPHIA_DECODER_H */
