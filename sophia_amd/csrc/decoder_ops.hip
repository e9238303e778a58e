// Element-wise and depth-mixing kernels of the hybrid decoder around the KDA
// mixer (the layers between the mixers):
//
//  * attn_res_mix_kernel -- AttentionResidualMixer.forward
//    (ml/runtime/model/blocks.py:30-48): a softmax over the depth axis of
//    [completed blocks..., partial] with scores RMSNorm(value) . query,
//    then the weighted sum of the values.  With r_b = rsqrt(mean(v_b^2) + eps),
//    score_b = r_b * sum_e v_b[e] * (w_norm[e] * q[e]), so one pass over the
//    values gives every score and a second pass (L2-resident) the mix; the
//    values are never concatenated or normalised in memory.
//  * situ_glu_kernel -- the SiTU-GLU hidden of FeedForward.forward
//    (blocks.py:23-27): h = cg tanh(g/cg) sigmoid(g) * cu tanh(u/cu) from the
//    fused [gate | up] projection, in one pass.
//
// Both compute in fp32 and round once on output (the reference rounds the
// normalised keys, the softmax weights and the products to the activation
// dtype in between).
#include "common.hpp"

#include "../../include/sophia_decoder.h"

namespace sophia {
namespace {

constexpr int kMaxDepth = 16;           // completed blocks + partial
constexpr int kMixChunksPerThread = 2;  // 8-element chunks per thread: dim <= 16 * 256

// Eight consecutive elements of a row as floats.
__device__ __forceinline__ void load8(const void *base, int64_t idx, int dtype, float (&v)[8]) {
  if (dtype == SOPHIA_DTYPE_BF16) {
    const u4 w = *reinterpret_cast<const u4 *>(static_cast<const uint16_t *>(base) + idx);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = __uint_as_float(w[i] << 16);
      v[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    }
  } else {
    const f4 a = *reinterpret_cast<const f4 *>(static_cast<const float *>(base) + idx);
    const f4 b = *reinterpret_cast<const f4 *>(static_cast<const float *>(base) + idx + 4);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[i] = a[i];
      v[4 + i] = b[i];
    }
  }
}

__device__ __forceinline__ void store8(void *base, int64_t idx, int dtype, const float (&v)[8]) {
  if (dtype == SOPHIA_DTYPE_BF16) {
    u4 w;
#pragma unroll
    for (int i = 0; i < 4; ++i) w[i] = pack_bf16x2(v[2 * i], v[2 * i + 1]);
    *reinterpret_cast<u4 *>(static_cast<uint16_t *>(base) + idx) = w;
  } else {
    *reinterpret_cast<f4 *>(static_cast<float *>(base) + idx) = f4{v[0], v[1], v[2], v[3]};
    *reinterpret_cast<f4 *>(static_cast<float *>(base) + idx + 4) = f4{v[4], v[5], v[6], v[7]};
  }
}

struct MixArgs {
  const void *partial;
  int64_t partial_stride;
  const void *completed;
  int64_t completed_row_stride, completed_block_stride;
  int n_blocks;
  const float *norm_w, *query_w;
  float eps;
  const float *out_norm_w;  // NULL: plain mix; else RMSNorm(mix; out_norm_w, out_eps)
  float out_eps;
  void *out;
  int64_t out_stride;
  int dim;
  int dtype;
};

__device__ __forceinline__ const void *depth_value(const MixArgs &a, int64_t row, int b) {
  // b < n_blocks: completed block b; b == n_blocks: the partial block.
  const int esz = a.dtype == SOPHIA_DTYPE_BF16 ? 2 : 4;
  if (b < a.n_blocks)
    return static_cast<const uint8_t *>(a.completed) +
           (row * a.completed_row_stride + static_cast<int64_t>(b) * a.completed_block_stride) * esz;
  return static_cast<const uint8_t *>(a.partial) + row * a.partial_stride * esz;
}

// One row per workgroup; thread t owns the 8-element chunks t and t + blockDim
// (dim <= 16 * blockDim).  DEPTH = completed blocks + 1, a template argument
// so that the per-block sums stay in registers.
template <int DEPTH>
__global__ __launch_bounds__(256) void attn_res_mix_kernel(MixArgs a) {
  __shared__ float red[2 * DEPTH + 1][4];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int nw = blockDim.x >> 6;
  const int64_t row = blockIdx.x;
  const int chunks = a.dim >> 3;
  // Pass 1: per depth block, sum v^2 and v . (w_norm * q) over this thread's chunks.
  float ss[DEPTH], dq[DEPTH];
#pragma unroll
  for (int b = 0; b < DEPTH; ++b) ss[b] = dq[b] = 0.f;
#pragma unroll
  for (int k = 0; k < kMixChunksPerThread; ++k) {
    const int c = tid + k * blockDim.x;
    if (c < chunks) {
      float wq[8];
      const f4 n0 = *reinterpret_cast<const f4 *>(a.norm_w + 8 * c);
      const f4 n1 = *reinterpret_cast<const f4 *>(a.norm_w + 8 * c + 4);
      const f4 q0 = *reinterpret_cast<const f4 *>(a.query_w + 8 * c);
      const f4 q1 = *reinterpret_cast<const f4 *>(a.query_w + 8 * c + 4);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        wq[i] = n0[i] * q0[i];
        wq[4 + i] = n1[i] * q1[i];
      }
#pragma unroll
      for (int b = 0; b < DEPTH; ++b) {
        float v[8];
        load8(depth_value(a, row, b), 8 * c, a.dtype, v);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          ss[b] = fmaf(v[i], v[i], ss[b]);
          dq[b] = fmaf(v[i], wq[i], dq[b]);
        }
      }
    }
  }
#pragma unroll
  for (int b = 0; b < DEPTH; ++b) {
    const float s2 = wave_sum(ss[b]);
    const float d = wave_sum(dq[b]);
    if (lane == 0) {
      red[2 * b][wave] = s2;
      red[2 * b + 1][wave] = d;
    }
  }
  lds_barrier();
  // Scores and softmax over the depth axis, in every thread.
  float p[DEPTH];
  float mx = -INFINITY;
#pragma unroll
  for (int b = 0; b < DEPTH; ++b) {
    float s2 = 0.f, d = 0.f;
    for (int w = 0; w < nw; ++w) {
      s2 += red[2 * b][w];
      d += red[2 * b + 1][w];
    }
    p[b] = d * rsqrtf(s2 / static_cast<float>(a.dim) + a.eps);
    mx = fmaxf(mx, p[b]);
  }
  float z = 0.f;
#pragma unroll
  for (int b = 0; b < DEPTH; ++b) {
    p[b] = __expf(p[b] - mx);
    z += p[b];
  }
  const float rz = 1.0f / z;
#pragma unroll
  for (int b = 0; b < DEPTH; ++b) p[b] *= rz;
  // Pass 2: the weighted sum (the values were just read by this thread: cache hits).
  float o[kMixChunksPerThread][8];
  float sq = 0.f;
#pragma unroll
  for (int k = 0; k < kMixChunksPerThread; ++k) {
    const int c = tid + k * blockDim.x;
#pragma unroll
    for (int i = 0; i < 8; ++i) o[k][i] = 0.f;
    if (c < chunks) {
#pragma unroll
      for (int b = 0; b < DEPTH; ++b) {
        float v[8];
        load8(depth_value(a, row, b), 8 * c, a.dtype, v);
#pragma unroll
        for (int i = 0; i < 8; ++i) o[k][i] = fmaf(p[b], v[i], o[k][i]);
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) sq = fmaf(o[k][i], o[k][i], sq);
    }
  }
  if (a.out_norm_w != nullptr) {  // uniform over the grid
    sq = wave_sum(sq);
    if (lane == 0) red[2 * DEPTH][wave] = sq;
    lds_barrier();
    float tot = 0.f;
    for (int w = 0; w < nw; ++w) tot += red[2 * DEPTH][w];
    const float r = rsqrtf(tot / static_cast<float>(a.dim) + a.out_eps);
#pragma unroll
    for (int k = 0; k < kMixChunksPerThread; ++k) {
      const int c = tid + k * blockDim.x;
      if (c < chunks) {
        const f4 w0 = *reinterpret_cast<const f4 *>(a.out_norm_w + 8 * c);
        const f4 w1 = *reinterpret_cast<const f4 *>(a.out_norm_w + 8 * c + 4);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          o[k][i] *= r * w0[i];
          o[k][4 + i] *= r * w1[i];
        }
      }
    }
  }
  uint8_t *dst = static_cast<uint8_t *>(a.out) + row * a.out_stride * (a.dtype == SOPHIA_DTYPE_BF16 ? 2 : 4);
#pragma unroll
  for (int k = 0; k < kMixChunksPerThread; ++k) {
    const int c = tid + k * blockDim.x;
    if (c < chunks) store8(dst, 8 * c, a.dtype, o[k]);
  }
}

// tanh from one exponential: t = e^{-2|x|}, tanh(x) = sign(x) (1 - t) / (1 + t);
// below |x| = 1/8, where 1 - t cancels, the Taylor series
// x (1 - x^2/3 + 2x^4/15 - 17x^6/315) (truncation below 2e-9 relative).
__device__ __forceinline__ float tanh_f(float x) {
  const float ax = fabsf(x);
  const float t = __expf(-2.0f * ax);
  const float big = (1.0f - t) / (1.0f + t);
  const float x2 = x * x;
  const float small = ax * fmaf(x2, fmaf(x2, fmaf(x2, -17.0f / 315.0f, 2.0f / 15.0f), -1.0f / 3.0f), 1.0f);
  return copysignf(ax < 0.125f ? small : big, x);
}

__global__ __launch_bounds__(256) void situ_glu_kernel(const void *gu, int64_t gu_stride, void *h, int64_t h_stride,
                                                       int64_t rows, int hidden, float gate_cap, float up_cap,
                                                       int dtype) {
  const int chunks = hidden / 8;
  const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t row = t / chunks;
  const int c = static_cast<int>(t % chunks);
  if (row >= rows) return;
  const int esz = dtype == SOPHIA_DTYPE_BF16 ? 2 : 4;
  const uint8_t *base = static_cast<const uint8_t *>(gu) + row * gu_stride * esz;
  float g[8], u[8], o[8];
  load8(base, 8 * c, dtype, g);
  load8(base, hidden + 8 * c, dtype, u);
  const float rcg = 1.0f / gate_cap, rcu = 1.0f / up_cap;
#pragma unroll
  for (int i = 0; i < 8; ++i)
    o[i] = gate_cap * tanh_f(g[i] * rcg) * sigmoid_f(g[i]) * (up_cap * tanh_f(u[i] * rcu));
  store8(static_cast<uint8_t *>(h) + row * h_stride * esz, 8 * c, dtype, o);
}

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

}  // namespace
}  // namespace sophia

using namespace sophia;

extern "C" int sophia_attn_res_mix(const void *partial, int64_t partial_stride, const void *completed,
                                   int64_t completed_row_stride, int64_t completed_block_stride, int n_blocks,
                                   const float *norm_weight, const float *query_weight, float eps,
                                   const float *out_norm_weight, float out_eps, void *out, int64_t out_stride,
                                   int64_t rows, int dim, int dtype, void *stream) {
  SOPHIA_REQUIRE(dtype == SOPHIA_DTYPE_F32 || dtype == SOPHIA_DTYPE_BF16, "attn_res_mix: dtype %d not supported",
                 dtype);
  SOPHIA_REQUIRE(rows >= 0 && dim > 0 && dim % 8 == 0 && dim <= 8 * kMixChunksPerThread * 256,
                 "attn_res_mix: dim must be a positive multiple of 8, at most %d", 8 * kMixChunksPerThread * 256);
  SOPHIA_REQUIRE(n_blocks >= 0 && n_blocks < kMaxDepth, "attn_res_mix: n_blocks must be in [0, %d)", kMaxDepth);
  SOPHIA_REQUIRE(rows == 0 || (partial && norm_weight && query_weight && out && (n_blocks == 0 || completed)),
                 "attn_res_mix: NULL pointer");
  SOPHIA_REQUIRE(partial_stride % 8 == 0 && out_stride % 8 == 0 && completed_row_stride % 8 == 0 &&
                     completed_block_stride % 8 == 0,
                 "attn_res_mix: strides must be multiples of 8 elements");
  SOPHIA_REQUIRE(partial_stride >= dim && out_stride >= dim && (n_blocks == 0 || completed_block_stride >= dim),
                 "attn_res_mix: stride smaller than a row");
  SOPHIA_REQUIRE(aligned16(partial) && aligned16(out) && aligned16(norm_weight) && aligned16(query_weight) &&
                     aligned16(out_norm_weight) && (n_blocks == 0 || aligned16(completed)),
                 "attn_res_mix: pointers must be 16-byte aligned");
  SOPHIA_REQUIRE(rows <= 0x7fffffff, "attn_res_mix: too many rows");
  if (rows == 0) return SOPHIA_OK;
  MixArgs a{partial, partial_stride, completed, completed_row_stride, completed_block_stride, n_blocks, norm_weight,
            query_weight, eps, out_norm_weight, out_eps, out, out_stride, dim, dtype};
  const int chunks = dim / 8;
  const int per_thread = (chunks + 255) / 256;
  const int threads = ((chunks + per_thread - 1) / per_thread + 63) / 64 * 64;
  const dim3 grid(static_cast<unsigned>(rows)), block(threads);
  const hipStream_t st = static_cast<hipStream_t>(stream);
  switch (n_blocks + 1) {
#define SOPHIA_MIX_CASE(d) \
  case d: hipLaunchKernelGGL(attn_res_mix_kernel<d>, grid, block, 0, st, a); break;
    SOPHIA_MIX_CASE(1) SOPHIA_MIX_CASE(2) SOPHIA_MIX_CASE(3) SOPHIA_MIX_CASE(4)
    SOPHIA_MIX_CASE(5) SOPHIA_MIX_CASE(6) SOPHIA_MIX_CASE(7) SOPHIA_MIX_CASE(8)
    SOPHIA_MIX_CASE(9) SOPHIA_MIX_CASE(10) SOPHIA_MIX_CASE(11) SOPHIA_MIX_CASE(12)
    SOPHIA_MIX_CASE(13) SOPHIA_MIX_CASE(14) SOPHIA_MIX_CASE(15) SOPHIA_MIX_CASE(16)
#undef SOPHIA_MIX_CASE
  }
  return check_launch("attn_res_mix");
}

extern "C" int sophia_situ_glu(const void *gate_up, int64_t gate_up_stride, void *hidden_out, int64_t out_stride,
                               int64_t rows, int hidden, float gate_softcap, float up_softcap, int dtype,
                               void *stream) {
  SOPHIA_REQUIRE(dtype == SOPHIA_DTYPE_F32 || dtype == SOPHIA_DTYPE_BF16, "situ_glu: dtype %d not supported", dtype);
  SOPHIA_REQUIRE(rows >= 0 && hidden > 0 && hidden % 8 == 0, "situ_glu: hidden must be a positive multiple of 8");
  SOPHIA_REQUIRE(rows == 0 || (gate_up && hidden_out), "situ_glu: NULL pointer");
  SOPHIA_REQUIRE(gate_up_stride % 8 == 0 && out_stride % 8 == 0 && gate_up_stride >= 2 * static_cast<int64_t>(hidden) &&
                     out_stride >= hidden,
                 "situ_glu: bad strides");
  SOPHIA_REQUIRE(gate_softcap > 0.f && up_softcap > 0.f, "situ_glu: soft caps must be positive");
  SOPHIA_REQUIRE(aligned16(gate_up) && aligned16(hidden_out), "situ_glu: pointers must be 16-byte aligned");
  if (rows == 0) return SOPHIA_OK;
  const int64_t threads = rows * (hidden / 8);
  const int64_t blocks = (threads + 255) / 256;
  SOPHIA_REQUIRE(blocks <= 0x7fffffff, "situ_glu: too many rows");
  hipLaunchKernelGGL(situ_glu_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), gate_up, gate_up_stride, hidden_out, out_stride, rows, hidden,
                     gate_softcap, up_softcap, dtype);
  return check_launch("situ_glu");
}
