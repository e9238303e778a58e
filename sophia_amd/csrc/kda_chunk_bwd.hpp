// Chunk-form backward of kda_chunk.hip, called by the backward entry point in
// kda_bwd.hip (sophia_kda_chunk_bwd), which adds dA_log and ddt_bias from the
// gradient of g.  Internal to the library: no C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

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
  // outputs: gradients of q, k, g (the gate's input, or the log-decay
  // itself without the gate in the kernel), v [total][H][128], of beta
  // [total][H] (all fp32) and of the initial states (or NULL)
  float *dq, *dk, *dg, *dbeta, *dv, *dh0;
};

// Scratch bytes chunk_bwd_run needs (256-byte aligned start).
size_t chunk_bwd_scratch_bytes(int64_t total_tokens, int n_seqs, int num_heads);

// Records of every (chunk, head), the forward states, the reverse chunk scan
// and the per-chunk gradients, on `stream`.  Returns a SOPHIA_* status.
int chunk_bwd_run(const ChunkBwdIO &io, void *scratch, hipStream_t stream);

}  // namespace sophia
