// Chunk-form backward of kda_chunk.hip, called by the backward entry point in
// kda_bwd.hip (sophia_kda_chunk_bwd), which adds dA_log and ddt_bias from the
// gradient of g.  Internal to the library: no C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "common.hpp"

namespace sophia {

struct ChunkBwdIO {
  // the forward's inputs, as sophia_kda_chunk_fwd takes them
  const void *q, *k, *v;
  int64_t qkv_stride;
  int qkv_dtype;
  const void *g;
  int64_t g_stride;
  int g_dtype;
  const void *beta;
  int64_t beta_stride;
  int beta_dtype;
  const float *A_log, *dt_bias;
  float scale, lb;
  unsigned flags;
  const int32_t *cu;
  int n_seqs;
  int64_t total;
  int num_heads;
  const float *h0;          // [n_seqs][H][128][128] or NULL
  // the gradients coming in
  const void *dout;
  int64_t do_stride;
  int do_dtype;
  const float *dht;         // [n_seqs][H][128][128] or NULL
  // outputs: gradients of q, k, v [total][H][128] (element type grad_dtype),
  // of g (the gate's input, or the log-decay itself without the gate in the
  // kernel) [total][H][128] and beta [total][H] (fp32), and of the initial
  // states (fp32, or NULL)
  void *dq, *dk;
  float *dg, *dbeta;
  void *dv;
  float *dh0;
  int grad_dtype;
};

// Rows outside every sequence (before cu[0], or from cu[n_seqs] on, both
// clamped into [0, total]) get zero gradients of q, k, v, g and beta: thread
// `t` of `threads` takes every threads-th element of those rows (usually
// none).
__device__ __forceinline__ void zero_rows_outside(const int32_t *cu, int n_seqs, int64_t total, int num_heads,
                                                  void *dq, void *dk, void *dv, int grad_dtype, float *dg,
                                                  float *dbeta, int64_t t, int64_t threads) {
  const int64_t lo = cu[0] < 0 ? 0 : (cu[0] > total ? total : cu[0]);
  const int64_t hi = cu[n_seqs] < lo ? lo : (cu[n_seqs] > total ? total : cu[n_seqs]);
  const int64_t per_row = static_cast<int64_t>(num_heads) * 128;
  const int64_t outside = (lo + (total - hi)) * per_row;
  for (int64_t i = t; i < outside; i += threads) {
    const int64_t r = i / per_row;
    const int64_t row = r < lo ? r : hi + (r - lo);
    const int64_t e = row * per_row + (i - r * per_row);
    store_elem(dq, e, grad_dtype, 0.f);
    store_elem(dk, e, grad_dtype, 0.f);
    store_elem(dv, e, grad_dtype, 0.f);
    dg[e] = 0.f;
    if (i - r * per_row < num_heads) dbeta[row * num_heads + (i - r * per_row)] = 0.f;
  }
}

// Scratch bytes chunk_bwd_run needs (256-byte aligned start).
size_t chunk_bwd_scratch_bytes(int64_t total_tokens, int n_seqs, int num_heads);

// Records of every (chunk, head), the forward states, the reverse chunk scan
// and the per-chunk gradients, on `stream`; also the zero gradients of rows
// outside every sequence.  Returns a SOPHIA_* status.
int chunk_bwd_run(const ChunkBwdIO &io, void *scratch, hipStream_t stream);

}  // namespace sophia
