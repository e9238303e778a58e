// KDA recurrent decode step: one token for each of `batch` sequences.
//
// Replaces fla.ops.kda.fused_recurrent_kda as called by SophiaKDA._run_kda
// (ml/runtime/model/attention.py:330-348).  Per (sequence, head), with the
// fp32 state S[k][v] (128 x 128):
//   S' = Diag(alpha) S + k u^T,   u = beta * (v - (Diag(alpha) S)^T k)
//   o  = S'^T q = (Diag(alpha) S)^T q + (q . k) u
// (the per-token update of _reference_kda, attention.py:288-293, rearranged
// so that one pass over S yields both reductions and the new state).
//
// HBM-bound: the state is 64 KiB per (sequence, head) and is read once and
// written once, in place.  One 256-thread work-group owns one (sequence,
// head): thread t holds columns 4*(t%32) .. +3 of rows (t/32) + 8*r,
// r = 0..15, so each wavefront load/store instruction moves two adjacent
// 512-byte rows.  The two column reductions go through the wavefront
// halves (xor-32 shuffle) and 4 x 128 floats of LDS.
#include "common.hpp"

namespace sophia {
namespace {

constexpr int kD = 128;
constexpr int kThreads = 256;
constexpr int kRowsPerThread = kD / 8;

__global__ __launch_bounds__(kThreads) void kda_decode_kernel(
    const void *__restrict__ q, const void *__restrict__ k, const void *__restrict__ v,
    int64_t qkv_stride, int qkv_dtype, const void *__restrict__ g, int64_t g_stride, int g_dtype,
    const void *__restrict__ beta, int64_t beta_stride, int beta_dtype,
    const float *__restrict__ A_log, const float *__restrict__ dt_bias, float scale, float lb,
    unsigned flags, float *__restrict__ state, int n_slots, const int32_t *__restrict__ slots,
    int read_state, int num_heads, void *__restrict__ o, int64_t o_stride) {
  const int h = blockIdx.x;
  const int b = blockIdx.y;
  const int t = threadIdx.x;
  const int lane = t & 63;
  const int wave = t >> 6;
  const int cg = t & 31;         // column group: columns 4cg .. 4cg+3
  const int rg = t >> 5;         // row group: rows rg + 8r

  __shared__ float s_q[kD], s_k[kD], s_a[kD], s_v[kD];
  __shared__ float s_red[4][3];
  __shared__ float s_p[4][kD], s_r[4][kD];
  __shared__ float s_u[kD];

  const int slot = slots ? slots[b] : b;
  if (slot < 0 || slot >= n_slots) {  // no cache slot: output 0, no state touched
    if (t < kD)
      store_elem(o, static_cast<int64_t>(b) * o_stride + static_cast<int64_t>(h) * kD + t,
                 qkv_dtype, 0.f);
    return;
  }
  float *S = state + (static_cast<int64_t>(slot) * num_heads + h) * kD * kD;

  // Issue the state loads first: they do not depend on the token prologue.
  f4 st[kRowsPerThread];
  if (read_state) {
#pragma unroll
    for (int r = 0; r < kRowsPerThread; ++r)
      st[r] = __builtin_nontemporal_load(
          reinterpret_cast<const f4 *>(S + (rg + 8 * r) * kD + 4 * cg));
  } else {
#pragma unroll
    for (int r = 0; r < kRowsPerThread; ++r) st[r] = f4{0.f, 0.f, 0.f, 0.f};
  }

  // Token prologue: threads 0..127 own one key/value channel each.
  const int64_t row = static_cast<int64_t>(b) * qkv_stride + static_cast<int64_t>(h) * kD;
  float qv = 0.f, kv = 0.f;
  if (t < kD) {
    qv = load_elem(q, row + t, qkv_dtype);
    kv = load_elem(k, row + t, qkv_dtype);
    float gv = load_elem(g, static_cast<int64_t>(b) * g_stride + static_cast<int64_t>(h) * kD + t,
                         g_dtype);
    if (flags & SOPHIA_KDA_GATE_IN_KERNEL) gv = kda_log_decay(gv, __expf(A_log[h]), dt_bias[h * kD + t], lb);
    s_a[t] = __expf(gv);
    s_v[t] = load_elem(v, row + t, qkv_dtype);
  }
  float sq = wave_sum(qv * qv), sk = wave_sum(kv * kv), sqk = wave_sum(qv * kv);
  if (lane == 0) {
    s_red[wave][0] = sq;
    s_red[wave][1] = sk;
    s_red[wave][2] = sqk;
  }
  lds_barrier();
  float qs = scale, ks = 1.f;
  if (flags & SOPHIA_KDA_QK_L2NORM) {
    const float nq = sqrtf(s_red[0][0] + s_red[1][0]);
    const float nk = sqrtf(s_red[0][1] + s_red[1][1]);
    qs = scale / fmaxf(nq, 1e-12f);
    ks = 1.f / fmaxf(nk, 1e-12f);
  }
  const float qk = (s_red[0][2] + s_red[1][2]) * qs * ks;
  float bt = load_elem(beta, static_cast<int64_t>(b) * beta_stride + h, beta_dtype);
  if (flags & SOPHIA_KDA_BETA_SIGMOID) bt = sigmoid_f(bt);
  if (t < kD) {
    s_q[t] = qv * qs;
    s_k[t] = kv * ks;
  }
  lds_barrier();

  // Decay the held rows and form the two partial column reductions.
  f4 p = {0.f, 0.f, 0.f, 0.f}, rq = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int r = 0; r < kRowsPerThread; ++r) {
    const int i = rg + 8 * r;
    const float a = s_a[i];
    st[r] *= a;
    p += s_k[i] * st[r];
    rq += s_q[i] * st[r];
  }
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    p[c] += __shfl_xor(p[c], 32, 64);
    rq[c] += __shfl_xor(rq[c], 32, 64);
  }
  if ((lane & 32) == 0) {
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      s_p[wave][4 * cg + c] = p[c];
      s_r[wave][4 * cg + c] = rq[c];
    }
  }
  lds_barrier();
  if (t < kD) {
    const float pj = s_p[0][t] + s_p[1][t] + s_p[2][t] + s_p[3][t];
    const float rj = s_r[0][t] + s_r[1][t] + s_r[2][t] + s_r[3][t];
    const float u = bt * (s_v[t] - pj);
    s_u[t] = u;
    store_elem(o, static_cast<int64_t>(b) * o_stride + static_cast<int64_t>(h) * kD + t, qkv_dtype,
               rj + qk * u);
  }
  lds_barrier();
  const f4 u4v = *reinterpret_cast<const f4 *>(&s_u[4 * cg]);
#pragma unroll
  for (int r = 0; r < kRowsPerThread; ++r) {
    const int i = rg + 8 * r;
    f4 nv = st[r] + s_k[i] * u4v;
    __builtin_nontemporal_store(nv, reinterpret_cast<f4 *>(S + i * kD + 4 * cg));
  }
}

}  // namespace
}  // namespace sophia

using namespace sophia;

extern "C" int sophia_kda_decode_step(const void *q, const void *k, const void *v,
                                      int64_t qkv_row_stride, int qkv_dtype, const void *g,
                                      int64_t g_row_stride, int g_dtype, const void *beta,
                                      int64_t beta_row_stride, int beta_dtype, const float *A_log,
                                      const float *dt_bias, float scale, float lower_bound,
                                      unsigned flags, float *state, int n_state_slots,
                                      const int32_t *state_slots, int read_state, int batch,
                                      int num_heads, int head_dim,
                                      void *o, int64_t o_row_stride, void *stream) {
  SOPHIA_REQUIRE(head_dim == kD, "kda_decode_step: head_dim must be 128 (got %d)", head_dim);
  SOPHIA_REQUIRE(batch > 0 && batch <= 65535 && num_heads > 0,
                 "kda_decode_step: batch must be 1..65535 and num_heads > 0");
  SOPHIA_REQUIRE(qkv_dtype == SOPHIA_DTYPE_F32 || qkv_dtype == SOPHIA_DTYPE_BF16,
                 "kda_decode_step: qkv dtype %d not supported", qkv_dtype);
  SOPHIA_REQUIRE(g_dtype == SOPHIA_DTYPE_F32 || g_dtype == SOPHIA_DTYPE_BF16,
                 "kda_decode_step: g dtype %d not supported", g_dtype);
  SOPHIA_REQUIRE(beta_dtype == SOPHIA_DTYPE_F32 || beta_dtype == SOPHIA_DTYPE_BF16,
                 "kda_decode_step: beta dtype %d not supported", beta_dtype);
  SOPHIA_REQUIRE(q && k && v && g && beta && state && o, "kda_decode_step: NULL pointer");
  SOPHIA_REQUIRE(!(flags & SOPHIA_KDA_GATE_IN_KERNEL) || (A_log && dt_bias),
                 "kda_decode_step: gate in kernel needs A_log and dt_bias");
  SOPHIA_REQUIRE(qkv_row_stride >= (int64_t)num_heads * kD && g_row_stride >= (int64_t)num_heads * kD &&
                     beta_row_stride >= num_heads && o_row_stride >= (int64_t)num_heads * kD,
                 "kda_decode_step: row stride smaller than a row");
  SOPHIA_REQUIRE(((uintptr_t)state % 16) == 0, "kda_decode_step: state must be 16-byte aligned");
  SOPHIA_REQUIRE(n_state_slots >= 0, "kda_decode_step: n_state_slots must be >= 0");
  dim3 grid(num_heads, batch);
  hipLaunchKernelGGL(kda_decode_kernel, grid, dim3(kThreads), 0, static_cast<hipStream_t>(stream),
                     q, k, v, qkv_row_stride, qkv_dtype, g, g_row_stride, g_dtype, beta,
                     beta_row_stride, beta_dtype, A_log, dt_bias, scale, lower_bound, flags, state,
                     n_state_slots, state_slots, read_state, num_heads, o, o_row_stride);
  return check_launch("kda_decode_step");
}
