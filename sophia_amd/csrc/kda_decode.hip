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
// written once, in place.  Its value columns are independent, so two
// 256-thread work-groups share one (sequence, head), 64 columns each (32 KiB
// of state; 94 us instead of 97 us for the B = 256 step with one work-group
// of 128 columns, 99 us with four of 32: shorter work-groups drain the grid's
// tail sooner, and 68 instead of 96 VGPRs keep more of them resident).
// Thread t holds columns col0 + 4*(t%16) .. +3 of rows (t/16) + 16*r,
// r = 0..7, so each wavefront load/store instruction moves four 256-byte row
// pieces.  The two column reductions go through the wavefront (xor-16 and
// xor-32 shuffles) and 4 x 64 floats of LDS.
//
// The CONV variant also runs the one-token ShortConv of the head's q, k and v
// channels (attention.py:226-258 with T = 1: silu of the 4-tap causal conv
// over the cached 3-sample history, output rounded to the activation dtype)
// in its prologue, from the pre-conv projection rows, and writes the shifted
// history back: a decode layer is then one launch.  It keeps one work-group
// per (sequence, head) (128 value columns): with two, both would read a
// channel's history while one of them rewrites it.
#include "common.hpp"

namespace sophia {
namespace {

constexpr int kD = 128;
constexpr int kThreads = 256;
constexpr int kDecodeCols = 64;   // value columns per work-group

// Conv history samples per channel (kernel size 4).
constexpr int kConvHist = 3;

// Dtypes and the gate switch are template parameters so that the load batch
// below has no branches: the wave then waits for the token inputs alone
// (issued first) before the prologue, while the state is still in flight.

template <int QKV_DT, int G_DT, int B_DT, bool GATE, int NC, bool CONV>
__global__ __launch_bounds__(kThreads) void kda_decode_kernel(
    const void *__restrict__ q, const void *__restrict__ k, const void *__restrict__ v,
    int64_t qkv_stride, const void *__restrict__ g, int64_t g_stride,
    const void *__restrict__ beta, int64_t beta_stride,
    const float *__restrict__ A_log, const float *__restrict__ dt_bias, float scale, float lb,
    unsigned flags, float *__restrict__ state, int n_slots, const int32_t *__restrict__ slots,
    int read_state, int num_heads, void *__restrict__ o, int64_t o_stride,
    const float *__restrict__ conv_w, float *__restrict__ conv_state) {
  constexpr int CG = NC / 4;           // column groups of 4 columns
  constexpr int RG = kThreads / CG;    // row groups
  constexpr int RPT = kD / RG;         // rows per thread
  const int h = blockIdx.x / (kD / NC);
  const int col0 = (blockIdx.x % (kD / NC)) * NC;
  const int b = blockIdx.y;
  const int t = threadIdx.x;
  const int lane = t & 63;
  const int wave = t >> 6;
  const int cg = t % CG;         // column group: columns col0 + 4cg .. +3
  const int rg = t / CG;         // row group: rows rg + RG r

  __shared__ float s_q[kD], s_k[kD], s_a[kThreads], s_v[kThreads];
  __shared__ float s_red[4][3];
  __shared__ float s_p[4][NC], s_r[4][NC];
  __shared__ float s_u[NC];

  const int slot = slots ? slots[b] : b;
  if (slot < 0 || slot >= n_slots) {  // no cache slot: output 0, no state touched
    if (t < NC)
      store_elem(o, static_cast<int64_t>(b) * o_stride + static_cast<int64_t>(h) * kD + col0 + t,
                 QKV_DT, 0.f);
    return;
  }
  float *S = state + (static_cast<int64_t>(slot) * num_heads + h) * kD * kD;

  // Every load of the block is issued before the first use: the token inputs
  // as raw bits (a dtype conversion inside the dtype branch would make the
  // wave wait there), then the 64 KB state.  One memory round trip per block.
  const int64_t row = static_cast<int64_t>(b) * qkv_stride + static_cast<int64_t>(h) * kD;
  const int64_t grow = static_cast<int64_t>(b) * g_stride + static_cast<int64_t>(h) * kD;
  const int c = t & (kD - 1);   // threads 128..255 load the same channels again
  const uint32_t raw_q = load_raw(q, row + c, QKV_DT);
  const uint32_t raw_k = load_raw(k, row + c, QKV_DT);
  const uint32_t raw_v = load_raw(v, row + c, QKV_DT);
  const uint32_t raw_g = load_raw(g, grow + c, G_DT);
  const uint32_t raw_b = load_raw(beta, static_cast<int64_t>(b) * beta_stride + h, B_DT);
  float alog = 0.f, bias = 0.f;
  if constexpr (GATE) {
    bias = dt_bias[h * kD + c];
    alog = A_log[h];
  }
  // Conv taps and history of channel c of q, k and v: channels
  // h*128 + c, inner + h*128 + c and 2*inner + h*128 + c of the fused
  // [3 * inner] layout (inner = num_heads * 128).
  const int64_t inner = static_cast<int64_t>(num_heads) * kD;
  const int64_t chq = static_cast<int64_t>(h) * kD + c;
  float *hist = nullptr;
  f4 wq, wk, wv;
  float hq[kConvHist], hk[kConvHist], hv[kConvHist];
  if constexpr (CONV) {
    hist = conv_state + static_cast<int64_t>(slot) * 3 * inner * kConvHist;
    wq = *reinterpret_cast<const f4 *>(conv_w + chq * 4);
    wk = *reinterpret_cast<const f4 *>(conv_w + (inner + chq) * 4);
    wv = *reinterpret_cast<const f4 *>(conv_w + (2 * inner + chq) * 4);
#pragma unroll
    for (int j = 0; j < kConvHist; ++j) {
      hq[j] = hist[chq * kConvHist + j];
      hk[j] = hist[(inner + chq) * kConvHist + j];
      hv[j] = hist[(2 * inner + chq) * kConvHist + j];
    }
  }
  // Compiler-only fence: keeps the token loads issued ahead of the state
  // loads (memory returns in issue order, and the prologue needs only them).
  asm volatile("" ::: "memory");
  // The state is loaded unconditionally (a branch here would make the wave
  // drain every load at the join) and replaced by zeros afterwards when the
  // incoming state is to be ignored.
  f4 st[RPT];
#pragma unroll
  for (int r = 0; r < RPT; ++r)
    st[r] = __builtin_nontemporal_load(reinterpret_cast<const f4 *>(S + (rg + RG * r) * kD + col0 + 4 * cg));
  __builtin_amdgcn_sched_barrier(0);

  // Token prologue: threads 0..127 own one key/value channel each.
  // Computed by every thread (selects, not branches: a load used only under
  // a branch would be sunk into it, behind the state loads).
  const bool own = t < kD;
  float xq = raw_to_f32(raw_q, QKV_DT), xk = raw_to_f32(raw_k, QKV_DT), xv = raw_to_f32(raw_v, QKV_DT);
  if constexpr (CONV) {
    // The step of short_conv_step_kernel: history cast to the input dtype,
    // acc = w[3] x + sum_j w[j] h[j], silu, rounded to the activation dtype.
    const auto conv1 = [&](const f4 &w, float (&hh)[kConvHist], float x) {
#pragma unroll
      for (int j = 0; j < kConvHist; ++j) hh[j] = read_state ? as_dtype(hh[j], QKV_DT) : 0.f;
      float acc = w[3] * x;
#pragma unroll
      for (int j = 0; j < kConvHist; ++j) acc = fmaf(w[j], hh[j], acc);
      return as_dtype(acc * sigmoid_f(acc), QKV_DT);
    };
    // conv1 leaves the rounded history in hq / hk / hv for the write below.
    xq = conv1(wq, hq, xq);
    xk = conv1(wk, hk, xk);
    xv = conv1(wv, hv, xv);
  }
  const float qv = own ? xq : 0.f;
  const float kv = own ? xk : 0.f;
  float gv = raw_to_f32(raw_g, G_DT);
  if constexpr (GATE) gv = kda_log_decay(gv, __expf(alog), bias, lb);
  const float av = __expf(gv);
  const float vv = xv;
  s_a[t] = av;   // threads 128..255 write the unused upper halves
  s_v[t] = vv;
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
  float bt = raw_to_f32(raw_b, B_DT);
  if (flags & SOPHIA_KDA_BETA_SIGMOID) bt = sigmoid_f(bt);
  if (t < kD) {
    s_q[t] = qv * qs;
    s_k[t] = kv * ks;
  }
  if constexpr (CONV) {
    // A full barrier (global memory too): every wave has read the conv
    // history before any wave rewrites it, and the compiler cannot move the
    // history stores above it.  Its wait for the state loads costs little:
    // the state is used right below.
    __syncthreads();
    if (own) {
      const float in_q = raw_to_f32(raw_q, QKV_DT), in_k = raw_to_f32(raw_k, QKV_DT);
      const float in_v = raw_to_f32(raw_v, QKV_DT);
      float *pq = hist + chq * kConvHist, *pk = hist + (inner + chq) * kConvHist;
      float *pv = hist + (2 * inner + chq) * kConvHist;
#pragma unroll
      for (int j = 0; j + 1 < kConvHist; ++j) {
        pq[j] = hq[j + 1];
        pk[j] = hk[j + 1];
        pv[j] = hv[j + 1];
      }
      pq[kConvHist - 1] = in_q;
      pk[kConvHist - 1] = in_k;
      pv[kConvHist - 1] = in_v;
    }
  } else {
    lds_barrier();
  }

  if (!read_state) {
#pragma unroll
    for (int r = 0; r < RPT; ++r) st[r] = f4{0.f, 0.f, 0.f, 0.f};
  }

  // Decay the held rows and form the two partial column reductions.
  f4 p = {0.f, 0.f, 0.f, 0.f}, rq = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int r = 0; r < RPT; ++r) {
    const int i = rg + RG * r;
    const float a = s_a[i];
    st[r] *= a;
    p += s_k[i] * st[r];
    rq += s_q[i] * st[r];
  }
#pragma unroll
  for (int m = CG; m < 64; m *= 2)
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      p[c] += __shfl_xor(p[c], m, 64);
      rq[c] += __shfl_xor(rq[c], m, 64);
    }
  if (lane < CG) {
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      s_p[wave][4 * cg + c] = p[c];
      s_r[wave][4 * cg + c] = rq[c];
    }
  }
  lds_barrier();
  if (t < NC) {
    const float pj = s_p[0][t] + s_p[1][t] + s_p[2][t] + s_p[3][t];
    const float rj = s_r[0][t] + s_r[1][t] + s_r[2][t] + s_r[3][t];
    const float u = bt * (s_v[col0 + t] - pj);
    s_u[t] = u;
    store_elem(o, static_cast<int64_t>(b) * o_stride + static_cast<int64_t>(h) * kD + col0 + t, QKV_DT,
               rj + qk * u);
  }
  lds_barrier();
  const f4 u4v = *reinterpret_cast<const f4 *>(&s_u[4 * cg]);
#pragma unroll
  for (int r = 0; r < RPT; ++r) {
    const int i = rg + RG * r;
    f4 nv = st[r] + s_k[i] * u4v;
    __builtin_nontemporal_store(nv, reinterpret_cast<f4 *>(S + i * kD + col0 + 4 * cg));
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
  dim3 grid(num_heads * (kD / kDecodeCols), batch);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const bool gate = (flags & SOPHIA_KDA_GATE_IN_KERNEL) != 0;
  const int key = (qkv_dtype == SOPHIA_DTYPE_BF16) * 8 + (g_dtype == SOPHIA_DTYPE_BF16) * 4 +
                  (beta_dtype == SOPHIA_DTYPE_BF16) * 2 + (gate ? 1 : 0);
#define SOPHIA_DECODE_CASE(KEY, QD, GD, BD, GT)                                                  \
  case KEY:                                                                                      \
    hipLaunchKernelGGL((kda_decode_kernel<QD, GD, BD, GT, kDecodeCols, false>), grid, dim3(kThreads), 0, st, q, \
                       k, v, qkv_row_stride, g, g_row_stride, beta, beta_row_stride, A_log, dt_bias,   \
                       scale, lower_bound, flags, state, n_state_slots, state_slots, read_state, \
                       num_heads, o, o_row_stride, nullptr, nullptr);                            \
    break;
  constexpr int F = SOPHIA_DTYPE_F32, B = SOPHIA_DTYPE_BF16;
  switch (key) {
    SOPHIA_DECODE_CASE(0, F, F, F, false)
    SOPHIA_DECODE_CASE(1, F, F, F, true)
    SOPHIA_DECODE_CASE(2, F, F, B, false)
    SOPHIA_DECODE_CASE(3, F, F, B, true)
    SOPHIA_DECODE_CASE(4, F, B, F, false)
    SOPHIA_DECODE_CASE(5, F, B, F, true)
    SOPHIA_DECODE_CASE(6, F, B, B, false)
    SOPHIA_DECODE_CASE(7, F, B, B, true)
    SOPHIA_DECODE_CASE(8, B, F, F, false)
    SOPHIA_DECODE_CASE(9, B, F, F, true)
    SOPHIA_DECODE_CASE(10, B, F, B, false)
    SOPHIA_DECODE_CASE(11, B, F, B, true)
    SOPHIA_DECODE_CASE(12, B, B, F, false)
    SOPHIA_DECODE_CASE(13, B, B, F, true)
    SOPHIA_DECODE_CASE(14, B, B, B, false)
    SOPHIA_DECODE_CASE(15, B, B, B, true)
  }
#undef SOPHIA_DECODE_CASE
  return check_launch("kda_decode_step");
}

extern "C" int sophia_kda_decode_conv_step(const void *x_q, const void *x_k, const void *x_v,
                                           int64_t x_row_stride, int qkv_dtype, const float *conv_weight,
                                           float *conv_state, int kernel_size, const void *g,
                                           int64_t g_row_stride, int g_dtype, const void *beta,
                                           int64_t beta_row_stride, int beta_dtype, const float *A_log,
                                           const float *dt_bias, float scale, float lower_bound,
                                           unsigned flags, float *state, int n_state_slots,
                                           const int32_t *state_slots, int read_state, int batch,
                                           int num_heads, int head_dim, void *o, int64_t o_row_stride,
                                           void *stream) {
  SOPHIA_REQUIRE(head_dim == kD, "kda_decode_conv_step: head_dim must be 128 (got %d)", head_dim);
  SOPHIA_REQUIRE(kernel_size == kConvHist + 1, "kda_decode_conv_step: kernel_size must be %d", kConvHist + 1);
  SOPHIA_REQUIRE(batch > 0 && batch <= 65535 && num_heads > 0,
                 "kda_decode_conv_step: batch must be 1..65535 and num_heads > 0");
  SOPHIA_REQUIRE(qkv_dtype == SOPHIA_DTYPE_F32 || qkv_dtype == SOPHIA_DTYPE_BF16,
                 "kda_decode_conv_step: qkv dtype %d not supported", qkv_dtype);
  SOPHIA_REQUIRE(g_dtype == SOPHIA_DTYPE_F32 || g_dtype == SOPHIA_DTYPE_BF16,
                 "kda_decode_conv_step: g dtype %d not supported", g_dtype);
  SOPHIA_REQUIRE(beta_dtype == SOPHIA_DTYPE_F32 || beta_dtype == SOPHIA_DTYPE_BF16,
                 "kda_decode_conv_step: beta dtype %d not supported", beta_dtype);
  SOPHIA_REQUIRE(x_q && x_k && x_v && g && beta && state && o && conv_weight && conv_state,
                 "kda_decode_conv_step: NULL pointer");
  SOPHIA_REQUIRE(!(flags & SOPHIA_KDA_GATE_IN_KERNEL) || (A_log && dt_bias),
                 "kda_decode_conv_step: gate in kernel needs A_log and dt_bias");
  SOPHIA_REQUIRE(x_row_stride >= (int64_t)num_heads * kD && g_row_stride >= (int64_t)num_heads * kD &&
                     beta_row_stride >= num_heads && o_row_stride >= (int64_t)num_heads * kD,
                 "kda_decode_conv_step: row stride smaller than a row");
  SOPHIA_REQUIRE(((uintptr_t)state % 16) == 0 && ((uintptr_t)conv_weight % 16) == 0,
                 "kda_decode_conv_step: state and conv_weight must be 16-byte aligned");
  SOPHIA_REQUIRE(n_state_slots >= 0, "kda_decode_conv_step: n_state_slots must be >= 0");
  dim3 grid(num_heads, batch);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const bool gate = (flags & SOPHIA_KDA_GATE_IN_KERNEL) != 0;
  const int key = (qkv_dtype == SOPHIA_DTYPE_BF16) * 8 + (g_dtype == SOPHIA_DTYPE_BF16) * 4 +
                  (beta_dtype == SOPHIA_DTYPE_BF16) * 2 + (gate ? 1 : 0);
#define SOPHIA_DECODE_CONV_CASE(KEY, QD, GD, BD, GT)                                             \
  case KEY:                                                                                      \
    hipLaunchKernelGGL((kda_decode_kernel<QD, GD, BD, GT, kD, true>), grid, dim3(kThreads), 0, st, x_q, x_k, \
                       x_v, x_row_stride, g, g_row_stride, beta, beta_row_stride, A_log, dt_bias, \
                       scale, lower_bound, flags, state, n_state_slots, state_slots, read_state, \
                       num_heads, o, o_row_stride, conv_weight, conv_state);                     \
    break;
  constexpr int F = SOPHIA_DTYPE_F32, B = SOPHIA_DTYPE_BF16;
  switch (key) {
    SOPHIA_DECODE_CONV_CASE(0, F, F, F, false)
    SOPHIA_DECODE_CONV_CASE(1, F, F, F, true)
    SOPHIA_DECODE_CONV_CASE(2, F, F, B, false)
    SOPHIA_DECODE_CONV_CASE(3, F, F, B, true)
    SOPHIA_DECODE_CONV_CASE(4, F, B, F, false)
    SOPHIA_DECODE_CONV_CASE(5, F, B, F, true)
    SOPHIA_DECODE_CONV_CASE(6, F, B, B, false)
    SOPHIA_DECODE_CONV_CASE(7, F, B, B, true)
    SOPHIA_DECODE_CONV_CASE(8, B, F, F, false)
    SOPHIA_DECODE_CONV_CASE(9, B, F, F, true)
    SOPHIA_DECODE_CONV_CASE(10, B, F, B, false)
    SOPHIA_DECODE_CONV_CASE(11, B, F, B, true)
    SOPHIA_DECODE_CONV_CASE(12, B, B, F, false)
    SOPHIA_DECODE_CONV_CASE(13, B, B, F, true)
    SOPHIA_DECODE_CONV_CASE(14, B, B, B, false)
    SOPHIA_DECODE_CONV_CASE(15, B, B, B, true)
  }
#undef SOPHIA_DECODE_CONV_CASE
  return check_launch("kda_decode_conv_step");
}
