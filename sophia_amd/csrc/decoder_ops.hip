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
//  * gated_head_norm_kernel -- the gated outputs of the mixers: KDA's
//    RMSNorm(o per head) * sigmoid(gate) (ml/runtime/model/attention.py:
//    411-420) and MLA's o * sigmoid(gate) (attention.py:655-656).
//
// All compute in fp32 and round once on output (the reference rounds the
// normalised keys, the softmax weights and the products to the activation
// dtype in between).  Every kernel is bound by HBM traffic: each input byte
// is read once and each output byte written once.
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

__device__ __forceinline__ void unpack8(const u4 w, float (&v)[8]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    v[2 * i] = __uint_as_float(w[i] << 16);
    v[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
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

__device__ __forceinline__ bf8 bits_to_bf8(u4 w) { return __builtin_bit_cast(bf8, w); }

__device__ __forceinline__ u2 pack4_bf16(f4 v) {
  return u2{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
}

struct MixArgs {
  const void *partial;
  int64_t partial_stride;
  const void *residual;     // NULL, or added to the partial block first (then written to partial_out)
  int64_t residual_stride;
  void *partial_out;
  int64_t partial_out_stride;
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

// Chunk c of depth block b as floats; the partial block is partial + residual
// when a residual is given (an fp32 sum, rounded to bf16 for bf16 data, as the
// reference adds in the activation dtype).
__device__ __forceinline__ void load_depth(const MixArgs &a, int64_t row, int b, int c, int dtype, float (&v)[8]) {
  load8(depth_value(a, row, b), 8 * c, dtype, v);
  if (b == a.n_blocks && a.residual != nullptr) {
    float r[8];
    load8(static_cast<const uint8_t *>(a.residual) + row * a.residual_stride * (dtype == SOPHIA_DTYPE_BF16 ? 2 : 4),
          8 * c, dtype, r);
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] += r[i];
  }
}

// One row per workgroup; thread t owns the 8-element chunks t + k blockDim,
// k < CPT (dim <= 8 CPT blockDim).  DEPTH = completed blocks + 1.  Both are
// template arguments so that the per-block sums, and for bf16 the values
// themselves (4 VGPRs per chunk and block), stay in registers between the
// score pass and the mix pass; fp32 values are read again (cache hits).
template <int DEPTH, int CPT, bool BF16>
__global__ __launch_bounds__(256) void attn_res_mix_kernel(MixArgs a) {
  constexpr int kDt = BF16 ? SOPHIA_DTYPE_BF16 : SOPHIA_DTYPE_F32;
  __shared__ float red[2 * DEPTH + 1][4];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int nw = blockDim.x >> 6;
  const int64_t row = blockIdx.x;
  const int chunks = a.dim >> 3;
  const float inv_dim = 1.0f / static_cast<float>(a.dim);
  u4 raw[BF16 ? DEPTH : 1][CPT];
  float ss[DEPTH], dq[DEPTH];
#pragma unroll
  for (int b = 0; b < DEPTH; ++b) ss[b] = dq[b] = 0.f;
  // Pass 1: per depth block, sum v^2 and v . (w_norm * q) over this thread's chunks.
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    const int c = tid + k * blockDim.x;
    if (c < chunks) {
#pragma unroll
      for (int b = 0; b < DEPTH; ++b) {
        if constexpr (BF16)
          raw[b][k] = *reinterpret_cast<const u4 *>(static_cast<const uint16_t *>(depth_value(a, row, b)) + 8 * c);
      }
      if (a.residual != nullptr) {  // uniform: partial <- partial + residual, written out once
        float v[8];
        if constexpr (BF16) {
          float r[8];
          unpack8(raw[DEPTH - 1][k], v);
          load8(static_cast<const uint8_t *>(a.residual) + row * a.residual_stride * 2, 8 * c, kDt, r);
#pragma unroll
          for (int i = 0; i < 8; ++i) v[i] += r[i];
          u4 w;
#pragma unroll
          for (int i = 0; i < 4; ++i) w[i] = pack_bf16x2(v[2 * i], v[2 * i + 1]);
          raw[DEPTH - 1][k] = w;
        } else {
          load_depth(a, row, DEPTH - 1, c, kDt, v);
        }
        store8(static_cast<uint8_t *>(a.partial_out) + row * a.partial_out_stride * (BF16 ? 2 : 4), 8 * c, kDt, v);
      }
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
        if constexpr (BF16)
          unpack8(raw[b][k], v);
        else
          load_depth(a, row, b, c, kDt, v);
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
    p[b] = d * rsqrtf(s2 * inv_dim + a.eps);
    mx = fmaxf(mx, p[b]);
  }
  float z = 0.f;
#pragma unroll
  for (int b = 0; b < DEPTH; ++b) {
    p[b] = __expf(p[b] - mx);
    z += p[b];
  }
  const float rz = __builtin_amdgcn_rcpf(z);
#pragma unroll
  for (int b = 0; b < DEPTH; ++b) p[b] *= rz;
  // Pass 2: the weighted sum.
  float o[CPT][8];
  float sq = 0.f;
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    const int c = tid + k * blockDim.x;
#pragma unroll
    for (int i = 0; i < 8; ++i) o[k][i] = 0.f;
    if (c < chunks) {
#pragma unroll
      for (int b = 0; b < DEPTH; ++b) {
        float v[8];
        if constexpr (BF16)
          unpack8(raw[b][k], v);
        else
          load_depth(a, row, b, c, kDt, v);
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
    const float r = rsqrtf(tot * inv_dim + a.out_eps);
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
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
  uint8_t *dst = static_cast<uint8_t *>(a.out) + row * a.out_stride * (BF16 ? 2 : 4);
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    const int c = tid + k * blockDim.x;
    if (c < chunks) store8(dst, 8 * c, kDt, o[k]);
  }
}

// tanh(x) for x = |z| / cap >= 0 as a fraction num / den: with t = e^{-2x},
// (1 - t) / (1 + t); below x = 1/8, where 1 - t cancels, the Taylor series
// x (1 - x^2/3 + 2x^4/15 - 17x^6/315) over 1 (truncation below 2e-9
// relative).  t is returned for the sigmoid (cap 4: e^{-|z|} = t^2).
struct Frac {
  float num, den, t;
};

__device__ __forceinline__ Frac tanh_frac(float x) {
  constexpr float kM2Log2e = -2.0f * 1.44269504088896341f;
  const float t = __builtin_amdgcn_exp2f(kM2Log2e * x);
  const float x2 = x * x;
  const float poly = x * fmaf(x2, fmaf(x2, fmaf(x2, -17.0f / 315.0f, 2.0f / 15.0f), -1.0f / 3.0f), 1.0f);
  const bool small = x < 0.125f;
  return Frac{small ? poly : 1.0f - t, small ? 1.0f : 1.0f + t, t};
}

// One 8-element chunk per thread; a block covers 256 chunks of one row.
//   h = cg tanh(g/cg) sigmoid(g) * cu tanh(u/cu)
//     = cg cu sgn(g) sgn(u) num_g num_u s / (den_g den_u (1 + e))
// with e = e^{-|g|} <= 1 and s = 1 (g >= 0) or e (g < 0): every factor of the
// denominator lies in [1, 2], so one reciprocal serves the element.  With the
// reference's gate cap of 4 (CAP4), e = t_g^2 and no third exponential is
// needed.  Arguments are pre-scaled on the host: xg = -2 log2(e) / cg,
// xu = -2 log2(e) / cu (exponent factors) and rcg = 1 / cg, rcu = 1 / cu.
template <bool BF16, bool CAP4>
__global__ __launch_bounds__(256) void situ_glu_kernel(const void *gu, int64_t gu_stride, void *h, int64_t h_stride,
                                                       int hidden, int blocks_per_row, float rcg, float rcu,
                                                       float scale) {
  constexpr int kDt = BF16 ? SOPHIA_DTYPE_BF16 : SOPHIA_DTYPE_F32;
  const int row = blockIdx.x / blocks_per_row;  // scalar
  const int c = (blockIdx.x - row * blocks_per_row) * 256 + threadIdx.x;
  if (8 * c >= hidden) return;
  const uint8_t *base = static_cast<const uint8_t *>(gu) + static_cast<int64_t>(row) * gu_stride * (BF16 ? 2 : 4);
  float g[8], u[8], o[8];
  load8(base, 8 * c, kDt, g);
  load8(base, hidden + 8 * c, kDt, u);
  constexpr float kM2Log2e = -2.0f * 1.44269504088896341f;
  // With the up cap of 25 nearly every |u| / cu is below 1/8, where tanh_frac
  // takes its series: when that holds for the whole wavefront, the u side
  // skips the exponential and the selects (the same values either way).
  float umax = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) umax = fmaxf(umax, fabsf(u[i]) * rcu);
  const auto element = [&](auto u_series) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float ag = fabsf(g[i]);
      const Frac fg = tanh_frac(ag * rcg);
      Frac fu;
      if constexpr (decltype(u_series)::value) {
        const float x = fabsf(u[i]) * rcu, x2 = x * x;
        fu = Frac{x * fmaf(x2, fmaf(x2, fmaf(x2, -17.0f / 315.0f, 2.0f / 15.0f), -1.0f / 3.0f), 1.0f), 1.0f, 0.f};
      } else {
        fu = tanh_frac(fabsf(u[i]) * rcu);
      }
      float e;
      if constexpr (CAP4)
        e = fg.t * fg.t;
      else
        e = __builtin_amdgcn_exp2f(0.5f * kM2Log2e * ag);
      const float s = g[i] >= 0.f ? 1.0f : e;
      const float mag = scale * fg.num * fu.num * s * __builtin_amdgcn_rcpf(fg.den * fu.den * (1.0f + e));
      // sign of g times sign of u, as a flip of the sign bit
      o[i] = __uint_as_float(__float_as_uint(mag) ^ ((__float_as_uint(g[i]) ^ __float_as_uint(u[i])) & 0x80000000u));
    }
  };
  if (__all(umax < 0.125f))
    element(std::true_type{});
  else
    element(std::false_type{});
  store8(static_cast<uint8_t *>(h) + static_cast<int64_t>(row) * h_stride * (BF16 ? 2 : 4), 8 * c, kDt, o);
}

// Gated per-head output: y = (RMSNorm_head(o; w, eps) or o) * sigmoid(gate).
// One 8-element chunk per thread, G = head_dim / 8 consecutive lanes per head
// (G a power of two <= 64, so a head never straddles a wavefront); a block
// covers 256 chunks of one row.
struct GateArgs {
  const void *o;
  int64_t o_stride;
  int o_dtype;
  const void *gate;
  int64_t gate_stride;
  const float *norm_w;  // [head_dim] or NULL
  float eps;
  void *out;
  int64_t out_stride;
  int width;  // heads * head_dim
  int head_dim;
  int blocks_per_row;
  int dtype;  // of gate and out
};

__global__ __launch_bounds__(256) void gated_head_norm_kernel(GateArgs a) {
  const int row = blockIdx.x / a.blocks_per_row;  // scalar
  const int c = (blockIdx.x - row * a.blocks_per_row) * 256 + threadIdx.x;
  const int G = a.head_dim >> 3;
  const bool valid = 8 * c < a.width;  // whole heads are valid or not
  float o[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f}, g[8];
  if (valid) {
    load8(static_cast<const uint8_t *>(a.o) + static_cast<int64_t>(row) * a.o_stride * (a.o_dtype == SOPHIA_DTYPE_BF16 ? 2 : 4),
          8 * c, a.o_dtype, o);
    load8(static_cast<const uint8_t *>(a.gate) + static_cast<int64_t>(row) * a.gate_stride * (a.dtype == SOPHIA_DTYPE_BF16 ? 2 : 4),
          8 * c, a.dtype, g);
    if (a.o_dtype != a.dtype) {  // the reference casts o to the activation dtype first
#pragma unroll
      for (int i = 0; i < 8; ++i) o[i] = __uint_as_float(static_cast<uint32_t>(f32_to_bf16_bits(o[i])) << 16);
    }
  }
  if (a.norm_w != nullptr) {  // uniform
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) ss = fmaf(o[i], o[i], ss);
    for (int off = G >> 1; off > 0; off >>= 1) ss += __shfl_xor(ss, off, 64);
    const float r = rsqrtf(ss / static_cast<float>(a.head_dim) + a.eps);
    if (valid) {
      const int e0 = 8 * (c & (G - 1));
      const f4 w0 = *reinterpret_cast<const f4 *>(a.norm_w + e0);
      const f4 w1 = *reinterpret_cast<const f4 *>(a.norm_w + e0 + 4);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        o[i] *= r * w0[i];
        o[4 + i] *= r * w1[i];
      }
    }
  }
  if (!valid) return;
#pragma unroll
  for (int i = 0; i < 8; ++i)
    o[i] *= __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-1.44269504088896341f * g[i]));
  store8(static_cast<uint8_t *>(a.out) + static_cast<int64_t>(row) * a.out_stride * (a.dtype == SOPHIA_DTYPE_BF16 ? 2 : 4),
         8 * c, a.dtype, o);
}

// ---- gated head norm, backward (training) ---------------------------------------
// Per head vector o (rounded to the activation dtype as the forward does),
// r = rsqrt(mean(o^2) + eps), n = o r, s = sigmoid(gate):
//   with the norm:    y = n w s;  dgate = dy n w s (1 - s);  dw = sum_rows dy s n;
//                     dn = dy s w;  do = r (dn - n mean(dn n))
//   without it (MLA): y = o s;    dgate = dy o s (1 - s);  do = dy s.
// Each work-group takes kGnbRows rows of a 2048-column slice; its threads'
// dw sums are reduced through LDS in a fixed order into one partial per
// work-group, and a second kernel sums the partials in order (deterministic).
constexpr int kGnbRows = 16;

struct GateBwdArgs {
  const void *dy;
  int64_t dy_stride;
  const void *o;
  int64_t o_stride;
  int o_dtype;
  const void *gate;
  int64_t gate_stride;
  const float *norm_w;  // [head_dim] or NULL
  float eps;
  void *d_o;            // o's dtype
  int64_t do_stride;
  void *d_gate;         // the gate's dtype
  int64_t dg_stride;
  float *dw_part;       // [blocks][head_dim] (with the norm)
  float *dw;            // [head_dim]
  int rows;
  int width;
  int head_dim;
  int blocks_per_row;
  int n_blocks;
  int dtype;
};

__global__ __launch_bounds__(256) void gated_head_norm_bwd_kernel(GateBwdArgs a) {
  __shared__ float s_dw[256][9];
  const int rb = blockIdx.x / a.blocks_per_row;
  const int c = (blockIdx.x - rb * a.blocks_per_row) * 256 + threadIdx.x;
  const int G = a.head_dim >> 3;
  const bool valid = 8 * c < a.width;   // whole heads are valid or not
  const bool norm = a.norm_w != nullptr;
  const int e0 = 8 * (c & (G - 1));
  float w[8], dwacc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    w[i] = (norm && valid) ? a.norm_w[e0 + i] : 1.f;
    dwacc[i] = 0.f;
  }
  const int r_end = min(a.rows, (rb + 1) * kGnbRows);
  for (int row = rb * kGnbRows; row < r_end; ++row) {   // uniform over the work-group
    float o[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f}, g[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f},
          dy[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    if (valid) {
      load8(static_cast<const uint8_t *>(a.o) + static_cast<int64_t>(row) * a.o_stride * (a.o_dtype == SOPHIA_DTYPE_BF16 ? 2 : 4),
            8 * c, a.o_dtype, o);
      load8(static_cast<const uint8_t *>(a.gate) + static_cast<int64_t>(row) * a.gate_stride * (a.dtype == SOPHIA_DTYPE_BF16 ? 2 : 4),
            8 * c, a.dtype, g);
      load8(static_cast<const uint8_t *>(a.dy) + static_cast<int64_t>(row) * a.dy_stride * (a.dtype == SOPHIA_DTYPE_BF16 ? 2 : 4),
            8 * c, a.dtype, dy);
      if (a.o_dtype != a.dtype) {
#pragma unroll
        for (int i = 0; i < 8; ++i) o[i] = __uint_as_float(static_cast<uint32_t>(f32_to_bf16_bits(o[i])) << 16);
      }
    }
    float sg[8], d_o[8], d_g[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) sg[i] = 1.0f / (1.0f + __expf(-g[i]));
    if (norm) {   // uniform
      float ss = 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) ss = fmaf(o[i], o[i], ss);
      for (int off = G >> 1; off > 0; off >>= 1) ss += __shfl_xor(ss, off, 64);
      const float r = rsqrtf(ss / static_cast<float>(a.head_dim) + a.eps);
      float n[8], dn[8], dot = 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        n[i] = o[i] * r;
        dn[i] = dy[i] * sg[i] * w[i];
        dot = fmaf(dn[i], n[i], dot);
        d_g[i] = dy[i] * n[i] * w[i] * sg[i] * (1.f - sg[i]);
        dwacc[i] = fmaf(dy[i] * sg[i], n[i], dwacc[i]);
      }
      for (int off = G >> 1; off > 0; off >>= 1) dot += __shfl_xor(dot, off, 64);
      const float m = dot / static_cast<float>(a.head_dim);
#pragma unroll
      for (int i = 0; i < 8; ++i) d_o[i] = r * (dn[i] - n[i] * m);
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        d_o[i] = dy[i] * sg[i];
        d_g[i] = dy[i] * o[i] * sg[i] * (1.f - sg[i]);
      }
    }
    if (valid) {
      store8(static_cast<uint8_t *>(a.d_o) + static_cast<int64_t>(row) * a.do_stride * (a.o_dtype == SOPHIA_DTYPE_BF16 ? 2 : 4),
             8 * c, a.o_dtype, d_o);
      store8(static_cast<uint8_t *>(a.d_gate) + static_cast<int64_t>(row) * a.dg_stride * (a.dtype == SOPHIA_DTYPE_BF16 ? 2 : 4),
             8 * c, a.dtype, d_g);
    }
  }
  if (!norm) return;
  // threads t with the same t % G hold the same 8 weight positions
#pragma unroll
  for (int i = 0; i < 8; ++i) s_dw[threadIdx.x][i] = valid ? dwacc[i] : 0.f;
  __syncthreads();
  if (threadIdx.x < a.head_dim) {
    const int lane = threadIdx.x >> 3, i = threadIdx.x & 7;   // weight position 8 lane + i
    float acc = 0.f;
    for (int t = lane; t < 256; t += G) acc += s_dw[t][i];
    a.dw_part[static_cast<int64_t>(blockIdx.x) * a.head_dim + threadIdx.x] = acc;
  }
}

__global__ __launch_bounds__(256) void gated_head_norm_dw_reduce_kernel(GateBwdArgs a) {
  const int e = blockIdx.x * 256 + threadIdx.x;
  if (e >= a.head_dim) return;
  float acc = 0.f;
  for (int b = 0; b < a.n_blocks; ++b) acc += a.dw_part[static_cast<int64_t>(b) * a.head_dim + e];
  a.dw[e] = acc;
}

// ---------------------------------------------------------------------------
// Absorbed MLA decode attention over fp32 latent caches.
//
// One work-group (4 wavefronts) per (decode row, key split).  A wavefront takes
// 16-key tiles of its range in turn and, per tile, on bf16 MFMAs:
//   S^T[16 keys x 16 heads] = lat[16 x R] . qa^T          (R / 32 MFMAs, K = rank)
//   lat^T blocks for the value sum: D = lat . I_sel        (one MFMA per 16 ranks)
//   ctx[16 heads x 16 ranks] += P[16 x 16 keys] . lat      (16x16x16 MFMAs, K = keys)
// The accumulator layout of S^T (lane: head = lane % 16, keys 4 (lane / 16) + i)
// is exactly the A-operand layout of P for the 16x16x16 product, and the
// accumulator layout of lat . I_sel (lane: rank column, keys 4 (lane / 16) + i) is
// its B operand, so no value passes through LDS inside the loop.  Softmax is
// online (running max and sum per head); the four wavefronts merge through LDS
// at the end, and key splits, when there are several, in a second kernel.
struct MlaArgs {
  const void *qa;        // [rows, heads, R]
  int64_t qa_stride;     // elements between rows
  int qa_dtype;
  const float *latent;   // [slots, max_seq, R] fp32
  int64_t slot_stride;   // elements between slots
  int max_seq;
  int n_slots;
  const int32_t *slots;  // [rows]
  const int64_t *pos;    // [rows]: keys 0..pos are attended
  float scale;
  void *out;             // [rows, heads, R]
  int64_t out_stride;
  int out_dtype;
  float *part;           // [rows, splits, 16, R + 2] when splits > 1
  int heads;
  int splits;
};

__device__ __forceinline__ f4 mfma32(const bf8 &a, const bf8 &b, const f4 &c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ f4 mfma16(const bf4 &a, const bf4 &b, const f4 &c) {
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s4, a), __builtin_bit_cast(s4, b), c, 0, 0,
                                                    0);
}

// Keys of a row: 0 for an out-of-range slot (its output is then zero).
__device__ __forceinline__ int mla_keys(const MlaArgs &a, int row, int64_t &slot) {
  slot = a.slots[row];
  if (slot < 0 || slot >= a.n_slots) return 0;
  const int64_t p = a.pos[row];
  return static_cast<int>(p < 0 ? 0 : (p + 1 > a.max_seq ? a.max_seq : p + 1));
}

template <int R>
__global__ __launch_bounds__(256) void mla_decode_kernel(MlaArgs a) {
  constexpr int KS = R / 32, NT = R / 16;
  __shared__ float s_acc[4][16][R];
  __shared__ float s_ml[4][2][16];
  const int row = blockIdx.x, split = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int ln = lane & 15, g = lane >> 4;
  int64_t slot;
  const int n = mla_keys(a, row, slot);
  const int tiles = (n + 15) >> 4;
  const int per = (tiles + a.splits - 1) / a.splits;
  const int t0 = split * per, t1 = min(tiles, t0 + per);
  const float *lat = a.latent + slot * a.slot_stride;

  // qa^T as B operands (lane: head ln, ranks 32 ks + 8 g + j); heads >= a.heads are zero.
  bf8 qb[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    float v[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    if (ln < a.heads)
      load8(static_cast<const uint8_t *>(a.qa) +
                (static_cast<int64_t>(row) * a.qa_stride + static_cast<int64_t>(ln) * R) *
                    (a.qa_dtype == SOPHIA_DTYPE_BF16 ? 2 : 4),
            32 * ks + 8 * g, a.qa_dtype, v);
#pragma unroll
    for (int j = 0; j < 8; ++j) qb[ks][j] = static_cast<__bf16>(v[j]);
  }
  // Selection operands: I_h picks ranks 16 h + n of a 32-rank block.
  bf8 sel[2];
#pragma unroll
  for (int hf = 0; hf < 2; ++hf)
#pragma unroll
    for (int j = 0; j < 8; ++j)
      sel[hf][j] = static_cast<__bf16>((8 * g + j == 16 * hf + ln) ? 1.0f : 0.0f);

  f4 acc[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) acc[nt] = f4{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_run = 0.f;

  f4 raw[2][KS][2];
  auto load_tile = [&](int t, f4 (&dst)[KS][2]) {
    const int key = min(16 * t + ln, n - 1);  // rows past the end are read in bounds and masked
    const float *rp = lat + static_cast<int64_t>(key) * R + 8 * g;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      dst[ks][0] = *reinterpret_cast<const f4 *>(rp + 32 * ks);
      dst[ks][1] = *reinterpret_cast<const f4 *>(rp + 32 * ks + 4);
    }
  };
  int t = t0 + wave;
  if (t < t1) load_tile(t, raw[0]);
  for (; t < t1; t += 4) {
    if (t + 4 < t1) load_tile(t + 4, raw[1]);
    bf8 af[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        af[ks][j] = static_cast<__bf16>(raw[0][ks][0][j]);
        af[ks][4 + j] = static_cast<__bf16>(raw[0][ks][1][j]);
      }
    f4 st = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) st = mfma32(af[ks], qb[ks], st);
    // st[i] = score of key 16 t + 4 g + i for head ln.
    float p[4], mx = -INFINITY;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      p[i] = (16 * t + 4 * g + i < n) ? st[i] * a.scale : -INFINITY;
      mx = fmaxf(mx, p[i]);
    }
    mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const float m_new = fmaxf(m_run, mx);  // finite: every tile holds a key < n
    const float alpha = __expf(m_run - m_new);
    float ps = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      p[i] = __expf(p[i] - m_new);
      ps += p[i];
    }
    ps += __shfl_xor(ps, 16, 64);
    ps += __shfl_xor(ps, 32, 64);
    l_run = l_run * alpha + ps;
    m_run = m_new;
    // ctx rows of this lane are heads 4 g + i: their factors live in lanes 4 g + i.
    float al[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) al[i] = __shfl(alpha, 4 * g + i, 64);
    const bf4 pa = bf4{static_cast<__bf16>(p[0]), static_cast<__bf16>(p[1]), static_cast<__bf16>(p[2]),
                       static_cast<__bf16>(p[3])};
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      const f4 tr = mfma32(af[nt >> 1], sel[nt & 1], f4{0.f, 0.f, 0.f, 0.f});
      const bf4 lb = bf4{static_cast<__bf16>(tr[0]), static_cast<__bf16>(tr[1]), static_cast<__bf16>(tr[2]),
                         static_cast<__bf16>(tr[3])};
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[nt][i] *= al[i];
      acc[nt] = mfma16(pa, lb, acc[nt]);
    }
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      raw[0][ks][0] = raw[1][ks][0];
      raw[0][ks][1] = raw[1][ks][1];
    }
  }
  // Merge the four wavefronts: acc[nt][i] is ctx[head 4 g + i][rank 16 nt + ln].
#pragma unroll
  for (int nt = 0; nt < NT; ++nt)
#pragma unroll
    for (int i = 0; i < 4; ++i) s_acc[wave][4 * g + i][16 * nt + ln] = acc[nt][i];
  if (g == 0) {
    s_ml[wave][0][ln] = m_run;
    s_ml[wave][1][ln] = l_run;
  }
  __syncthreads();
  const int heads = a.splits > 1 ? 16 : a.heads;
  for (int idx = tid; idx < heads * R; idx += 256) {
    const int h = idx / R, r = idx - h * R;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < 4; ++w) M = fmaxf(M, s_ml[w][0][h]);
    float num = 0.f, den = 0.f;
    if (M != -INFINITY) {
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const float e = __expf(s_ml[w][0][h] - M);
        num = fmaf(e, s_acc[w][h][r], num);
        den = fmaf(e, s_ml[w][1][h], den);
      }
    }
    if (a.splits > 1) {
      float *pp = a.part + ((static_cast<int64_t>(row) * a.splits + split) * 16 + h) * (R + 2);
      pp[r] = num;
      if (r == 0) {
        pp[R] = M;
        pp[R + 1] = den;
      }
    } else {
      const float y = den > 0.f ? num / den : 0.f;
      const int64_t o = static_cast<int64_t>(row) * a.out_stride + static_cast<int64_t>(h) * R + r;
      if (a.out_dtype == SOPHIA_DTYPE_BF16)
        static_cast<uint16_t *>(a.out)[o] = f32_to_bf16_bits(y);
      else
        static_cast<float *>(a.out)[o] = y;
    }
  }
}

// Merge of the key splits of one row: ctx = sum_s e^{m_s - M} acc_s / sum_s e^{m_s - M} l_s.
template <int R>
__global__ __launch_bounds__(256) void mla_decode_merge_kernel(MlaArgs a) {
  const int row = blockIdx.x;
  for (int idx = threadIdx.x; idx < a.heads * R; idx += 256) {
    const int h = idx / R, r = idx - h * R;
    const float *pp = a.part + (static_cast<int64_t>(row) * a.splits * 16 + h) * (R + 2);
    const int64_t step = 16 * static_cast<int64_t>(R + 2);
    float M = -INFINITY;
    for (int s = 0; s < a.splits; ++s) M = fmaxf(M, pp[s * step + R]);
    float num = 0.f, den = 0.f;
    if (M != -INFINITY) {
      for (int s = 0; s < a.splits; ++s) {
        const float e = __expf(pp[s * step + R] - M);
        num = fmaf(e, pp[s * step + r], num);
        den = fmaf(e, pp[s * step + R + 1], den);
      }
    }
    const float y = den > 0.f ? num / den : 0.f;
    const int64_t o = static_cast<int64_t>(row) * a.out_stride + static_cast<int64_t>(h) * R + r;
    if (a.out_dtype == SOPHIA_DTYPE_BF16)
      static_cast<uint16_t *>(a.out)[o] = f32_to_bf16_bits(y);
    else
      static_cast<float *>(a.out)[o] = y;
  }
}

// ---------------------------------------------------------------------------
// Causal attention over packed sequences (the MLA prefill rows, head_dim 128).
// The queries of sequence s are rows cu[s]..cu[s+1] of q; its keys and values
// are rows cu_k[s]..cu_k[s+1] of k and v (cu_k == NULL: the same rows).  With
// more keys than queries, the queries are the last positions of the key range
// (a prefill that continues after cached tokens): query i sees keys
// 0 .. i + (keys - queries).
//
// One work-group (4 wavefronts) per (128-query block, head, sequence); a
// wavefront owns 32 queries.  Per 64-key block, K (row-major) and V (transposed,
// keys along rows) are staged in LDS by the four wavefronts, then each
// wavefront forms
//   S^T[keys x queries] = K . Q^T            (A = K rows from LDS, B = Q^T in registers)
//   O^T[d x queries]   += V^T . P^T          (A = V^T from LDS, B = P^T from the S^T tiles)
// with v_mfma_f32_16x16x32_bf16.  The S^T accumulators of two 16-key tiles pair
// into the B operand of the second product (k order 4g..4g+3, 16+4g..16+4g+3,
// matched by the V^T reads), and O^T puts 4 consecutive head dims of one query
// in a lane, so the softmax state is per lane and the stores are 8 bytes.  V is
// transposed on its way into LDS by products with a 0/1 selection matrix.
constexpr int kFaD = 128;          // head dim
constexpr int kFaQ = 128;          // queries per work-group
constexpr int kFaK = 64;           // keys per block
constexpr int kFaLdK = kFaD + 8;   // bf16 row stride of the K tile
constexpr int kFaLdV = kFaK + 8;   // bf16 row stride of the V^T tile

struct FaArgs {
  const uint16_t *q, *k, *v;       // bf16 rows: token t, head h at t * stride + h * 128
  int64_t q_stride, k_stride, v_stride;
  uint16_t *out;
  int64_t out_stride;
  const int32_t *cu;
  const int32_t *cu_k;             // key offsets (NULL: cu)
  int n_seqs;
  int64_t total;
  int64_t total_k;                 // rows of k and v
  int q_blocks;                    // 128-query blocks per sequence (of max_len)
  int heads;
  float scale_log2;                // softmax scale * log2(e)
};

__global__ __launch_bounds__(256, 2) void causal_attn_kernel(FaArgs a) {
  __shared__ __attribute__((aligned(16))) uint16_t sK[kFaK * kFaLdK];
  __shared__ __attribute__((aligned(16))) uint16_t sVt[kFaD * kFaLdV];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int ln = lane & 15, g = lane >> 4;
  // XCD-aware order: work-group b runs on XCD b % 8, and every query block of
  // one (sequence, head) gets the same b % 8, so its K and V rows are fetched
  // from HBM once and then served by that XCD's L2.  Heavy (late) query blocks
  // are dispatched first.
  const int b = blockIdx.x;
  const int r = b >> 3;
  const int pair = (r / a.q_blocks) * 8 + (b & 7);
  if (pair >= a.heads * a.n_seqs) return;
  const int h = pair % a.heads, sq = pair / a.heads;
  const int64_t start = iclamp64(a.cu[sq], 0, a.total);
  const int len = static_cast<int>(iclamp64(a.cu[sq + 1], start, a.total) - start);
  int64_t kstart = start;
  int klen = len;
  if (a.cu_k) {
    kstart = iclamp64(a.cu_k[sq], 0, a.total_k);
    klen = static_cast<int>(iclamp64(a.cu_k[sq + 1], kstart, a.total_k) - kstart);
  }
  const int q0 = (a.q_blocks - 1 - r % a.q_blocks) * kFaQ;
  if (q0 >= len) return;
  if (klen < len) {
    // Fewer keys than queries: no query can be placed at its own key, so the
    // sequence's output rows are defined as zeros (never left unwritten).
    const int rows = min(kFaQ, len - q0);
    for (int i = tid; i < rows * (kFaD / 4); i += 256) {
      const int64_t row = start + q0 + i / (kFaD / 4);
      *reinterpret_cast<u2 *>(a.out + row * a.out_stride + static_cast<int64_t>(h) * kFaD + 4 * (i % (kFaD / 4))) =
          u2{0u, 0u};
    }
    return;
  }
  const int off = klen - len;                     // position of query 0 among the keys
  const int kend = min(klen, q0 + off + kFaQ);    // keys needed by this work-group
  const int nkb = (kend + kFaK - 1) / kFaK;
  const int wq0 = q0 + 32 * w;                    // first query of this wavefront
  const int wq_last = min(wq0 + 31, len - 1) + off;  // position of the last query it stores

  // Q^T as B operands: lane (query ln of tile qt, g) holds dims 32 ks + 8 g .. +7.
  bf8 qf[2][4];
#pragma unroll
  for (int qt = 0; qt < 2; ++qt) {
    const int qi = min(wq0 + 16 * qt + ln, len - 1);
    const uint16_t *qp = a.q + (start + qi) * a.q_stride + static_cast<int64_t>(h) * kFaD + 8 * g;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) qf[qt][ks] = bits_to_bf8(*reinterpret_cast<const u4 *>(qp + 32 * ks));
  }
  bf8 sel[2];
#pragma unroll
  for (int hf = 0; hf < 2; ++hf)
#pragma unroll
    for (int j = 0; j < 8; ++j) sel[hf][j] = static_cast<__bf16>((8 * g + j == 16 * hf + ln) ? 1.0f : 0.0f);

  f4 ot[2][8];
#pragma unroll
  for (int qt = 0; qt < 2; ++qt)
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) ot[qt][dt] = f4{0.f, 0.f, 0.f, 0.f};
  float m_run[2] = {-INFINITY, -INFINITY}, l_run[2] = {0.f, 0.f};

  // This lane's K / V rows of a block: key 16 w + ln, dims 32 ks + 8 g .. +7.
  u4 kr[4], vr[4];
  auto load_block = [&](int kb) {
    const int key = min(kb * kFaK + 16 * w + ln, klen - 1);
    const uint16_t *kp = a.k + (kstart + key) * a.k_stride + static_cast<int64_t>(h) * kFaD + 8 * g;
    const uint16_t *vp = a.v + (kstart + key) * a.v_stride + static_cast<int64_t>(h) * kFaD + 8 * g;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      kr[ks] = *reinterpret_cast<const u4 *>(kp + 32 * ks);
      vr[ks] = *reinterpret_cast<const u4 *>(vp + 32 * ks);
    }
  };
  load_block(0);
  for (int kb = 0; kb < nkb; ++kb) {
    const int k0 = kb * kFaK;
    __syncthreads();  // the previous block's LDS reads are done
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      *reinterpret_cast<u4 *>(&sK[(16 * w + ln) * kFaLdK + 32 * ks + 8 * g]) = kr[ks];
#pragma unroll
      for (int hf = 0; hf < 2; ++hf) {
        const f4 tr = mfma32(bits_to_bf8(vr[ks]), sel[hf], f4{0.f, 0.f, 0.f, 0.f});
        // tr[i] = V[key 16 w + 4 g + i][dim 32 ks + 16 hf + ln]
        *reinterpret_cast<u2 *>(&sVt[(32 * ks + 16 * hf + ln) * kFaLdV + 16 * w + 4 * g]) = pack4_bf16(tr);
      }
    }
    __syncthreads();
    if (kb + 1 < nkb) load_block(kb + 1);
    if (k0 > wq_last) continue;  // every key of the block is after this wavefront's queries
    // Only a block that reaches past this wavefront's first query, or past the
    // last key, needs the causal / length mask (uniform over the wavefront).
    const bool masked = k0 + kFaK - 1 > wq0 + off || k0 + kFaK > klen;
    // S^T tiles: st[kt][qt][i] = score(key k0 + 16 kt + 4 g + i, query wq0 + 16 qt + ln).
    f4 st[4][2];
#pragma unroll
    for (int kt = 0; kt < 4; ++kt) {
      st[kt][0] = st[kt][1] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const bf8 kf = bits_to_bf8(*reinterpret_cast<const u4 *>(&sK[(16 * kt + ln) * kFaLdK + 32 * ks + 8 * g]));
        st[kt][0] = mfma32(kf, qf[0][ks], st[kt][0]);
        st[kt][1] = mfma32(kf, qf[1][ks], st[kt][1]);
      }
    }
    bf8 pf[2][2];  // [kp][qt]: P^T as B operands of the value product
#pragma unroll
    for (int qt = 0; qt < 2; ++qt) {
      // Raw scores here; the scale (times log2 e, > 0) enters through the
      // running max and one fused multiply-add per exponent.
      float mx = -INFINITY;
      if (masked) {
        const int qpos = wq0 + 16 * qt + ln + off;
#pragma unroll
        for (int kt = 0; kt < 4; ++kt)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int key = k0 + 16 * kt + 4 * g + i;
            const float sv = (key <= qpos && key < klen) ? st[kt][qt][i] : -INFINITY;
            st[kt][qt][i] = sv;
            mx = fmaxf(mx, sv);
          }
      } else {
#pragma unroll
        for (int kt = 0; kt < 4; ++kt)
#pragma unroll
          for (int i = 0; i < 4; ++i) mx = fmaxf(mx, st[kt][qt][i]);
      }
      mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
      const float m_new = fmaxf(m_run[qt], mx * a.scale_log2);
      // m_new is finite once key 0 has been seen, and key 0 is in the first block.
      const float alpha = __builtin_amdgcn_exp2f(m_run[qt] - m_new);
      float ps = 0.f;
#pragma unroll
      for (int kt = 0; kt < 4; ++kt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float pv = __builtin_amdgcn_exp2f(fmaf(st[kt][qt][i], a.scale_log2, -m_new));
          st[kt][qt][i] = pv;
          ps += pv;
        }
      ps += __shfl_xor(ps, 16, 64);
      ps += __shfl_xor(ps, 32, 64);
      l_run[qt] = l_run[qt] * alpha + ps;
      m_run[qt] = m_new;
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) ot[qt][dt] *= alpha;
#pragma unroll
      for (int kp = 0; kp < 2; ++kp)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          pf[kp][qt][i] = static_cast<__bf16>(st[2 * kp][qt][i]);
          pf[kp][qt][4 + i] = static_cast<__bf16>(st[2 * kp + 1][qt][i]);
        }
    }
    // O^T += V^T P^T: A = V^T rows dims 16 dt + ln, keys 32 kp + {4g..4g+3, 16+4g..16+4g+3}.
#pragma unroll
    for (int dt = 0; dt < 8; ++dt)
#pragma unroll
      for (int kp = 0; kp < 2; ++kp) {
        const uint16_t *vrow = &sVt[(16 * dt + ln) * kFaLdV + 32 * kp + 4 * g];
        const u2 lo = *reinterpret_cast<const u2 *>(vrow);
        const u2 hi = *reinterpret_cast<const u2 *>(vrow + 16);
        const bf8 vf = bits_to_bf8(u4{lo.x, lo.y, hi.x, hi.y});
        ot[0][dt] = mfma32(vf, pf[kp][0], ot[0][dt]);
        ot[1][dt] = mfma32(vf, pf[kp][1], ot[1][dt]);
      }
  }
  // ot[qt][dt][i] = O[query wq0 + 16 qt + ln][dim 16 dt + 4 g + i] before the 1 / l.
#pragma unroll
  for (int qt = 0; qt < 2; ++qt) {
    const int qi = wq0 + 16 * qt + ln;
    if (qi >= len) continue;
    const float rl = 1.0f / l_run[qt];
    uint16_t *op = a.out + (start + qi) * a.out_stride + static_cast<int64_t>(h) * kFaD + 4 * g;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) *reinterpret_cast<u2 *>(op + 16 * dt) = pack4_bf16(ot[qt][dt] * rl);
  }
}

// ---- MLA latent norms -----------------------------------------------------------
// The normalisations that follow MLA's down projections (attention.py:611-614):
// q_norm over the q_down output and kv_norm over the kv_down output, in place,
// and the normalised latent written into its latent-cache slot as fp32 (the
// value rounded to the activation dtype first, as latent.to(cache.dtype)
// converts it).  One wavefront per row: lanes [0, q_rank / 8) hold 8 elements
// of q each, the next kv_rank / 8 lanes 8 of the latent.  The norm weights are
// fp32 and rounded to the activation dtype, as RMSNorm.forward casts them.
struct MlaNormArgs {
  void *q;
  int64_t q_stride;
  void *kv;
  int64_t kv_stride;
  int q_rank, kv_rank, rows;
  const float *q_w, *kv_w;
  float q_eps, kv_eps;
  float *cache;                   // [n_slots][max_len][kv_rank] fp32, or NULL
  int n_slots, max_len;
  int n_prefill;                  // rows [0, n_prefill) are prefill rows
  const int32_t *seq_slot;        // rectangular prefill: row i -> (seq_slot[i / seq_len], i % seq_len)
  int seq_len;
  const int64_t *row_slot, *row_pos;             // else: (row_slot[i], row_pos[i])
  const int32_t *dec_slot;                       // decode row n_prefill + j -> (dec_slot[j], dec_pos[j])
  const int64_t *dec_pos;
};

template <bool BF16>
__global__ __launch_bounds__(256) void mla_latent_norm_kernel(MlaNormArgs a) {
  constexpr int kDt = BF16 ? SOPHIA_DTYPE_BF16 : SOPHIA_DTYPE_F32;
  constexpr int kEsz = BF16 ? 2 : 4;
  const int row = static_cast<int>(blockIdx.x) * 4 + static_cast<int>(threadIdx.x >> 6);
  if (row >= a.rows) return;  // uniform over the wavefront
  const int l = threadIdx.x & 63;
  const int qc = a.q_rank / 8, kc = a.kv_rank / 8;
  const bool isq = l < qc, iskv = l >= qc && l < qc + kc;
  const int c = isq ? l : l - qc;  // 8-element chunk within its part
  uint8_t *base = isq ? static_cast<uint8_t *>(a.q) + static_cast<int64_t>(row) * a.q_stride * kEsz
                      : static_cast<uint8_t *>(a.kv) + static_cast<int64_t>(row) * a.kv_stride * kEsz;
  float v[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  if (isq || iskv) load8(base, 8 * c, kDt, v);
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) ss = fmaf(v[i], v[i], ss);
  float sq = isq ? ss : 0.f, sk = iskv ? ss : 0.f;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    sq += __shfl_xor(sq, off, 64);
    sk += __shfl_xor(sk, off, 64);
  }
  if (!(isq || iskv)) return;
  const float r = isq ? rsqrtf(sq / static_cast<float>(a.q_rank) + a.q_eps)
                      : rsqrtf(sk / static_cast<float>(a.kv_rank) + a.kv_eps);
  const float *w = (isq ? a.q_w : a.kv_w) + 8 * c;
  float o[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) o[i] = as_dtype(v[i] * r * as_dtype(w[i], kDt), kDt);
  store8(base, 8 * c, kDt, o);
  if (!iskv || !a.cache) return;
  int64_t slot, pos;
  if (row < a.n_prefill) {
    if (a.seq_slot) {
      slot = a.seq_slot[row / a.seq_len];
      pos = row % a.seq_len;
    } else {
      slot = a.row_slot[row];
      pos = a.row_pos[row];
    }
  } else {
    slot = a.dec_slot[row - a.n_prefill];
    pos = a.dec_pos[row - a.n_prefill];
  }
  if (slot < 0 || slot >= a.n_slots || pos < 0 || pos >= a.max_len) return;
  f4 *dst = reinterpret_cast<f4 *>(a.cache + (slot * a.max_len + pos) * a.kv_rank + 8 * c);
  dst[0] = f4{o[0], o[1], o[2], o[3]};
  dst[1] = f4{o[4], o[5], o[6], o[7]};
}

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

}  // namespace
}  // namespace sophia

using namespace sophia;

extern "C" int sophia_attn_res_mix(const void *partial, int64_t partial_stride, const void *residual,
                                   int64_t residual_stride, void *partial_out, int64_t partial_out_stride,
                                   const void *completed,
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
  SOPHIA_REQUIRE(residual == nullptr || (partial_out != nullptr && aligned16(residual) && aligned16(partial_out) &&
                                          residual_stride % 8 == 0 && partial_out_stride % 8 == 0 &&
                                          residual_stride >= dim && partial_out_stride >= dim),
                 "attn_res_mix: a residual needs a partial_out; both 16-byte aligned with strides of 8");
  SOPHIA_REQUIRE(rows <= 0x7fffffff, "attn_res_mix: too many rows");
  if (rows == 0) return SOPHIA_OK;
  MixArgs a{partial, partial_stride, residual, residual_stride, partial_out, partial_out_stride, completed,
            completed_row_stride, completed_block_stride, n_blocks, norm_weight, query_weight, eps, out_norm_weight,
            out_eps, out, out_stride, dim, dtype};
  const int chunks = dim / 8;
  const int per_thread = (chunks + 255) / 256;
  const int threads = ((chunks + per_thread - 1) / per_thread + 63) / 64 * 64;
  const dim3 grid(static_cast<unsigned>(rows)), block(threads);
  const hipStream_t st = static_cast<hipStream_t>(stream);
  const int key = (n_blocks + 1) * 4 + (per_thread - 1) * 2 + (dtype == SOPHIA_DTYPE_BF16 ? 1 : 0);
  switch (key) {
#define SOPHIA_MIX_CASE(d, cpt, bf)                                                              \
  case d * 4 + (cpt - 1) * 2 + bf:                                                                \
    hipLaunchKernelGGL((attn_res_mix_kernel<d, cpt, bf != 0>), grid, block, 0, st, a);           \
    break;
#define SOPHIA_MIX_DEPTH(d) \
  SOPHIA_MIX_CASE(d, 1, 0) SOPHIA_MIX_CASE(d, 1, 1) SOPHIA_MIX_CASE(d, 2, 0) SOPHIA_MIX_CASE(d, 2, 1)
    SOPHIA_MIX_DEPTH(1) SOPHIA_MIX_DEPTH(2) SOPHIA_MIX_DEPTH(3) SOPHIA_MIX_DEPTH(4)
    SOPHIA_MIX_DEPTH(5) SOPHIA_MIX_DEPTH(6) SOPHIA_MIX_DEPTH(7) SOPHIA_MIX_DEPTH(8)
    SOPHIA_MIX_DEPTH(9) SOPHIA_MIX_DEPTH(10) SOPHIA_MIX_DEPTH(11) SOPHIA_MIX_DEPTH(12)
    SOPHIA_MIX_DEPTH(13) SOPHIA_MIX_DEPTH(14) SOPHIA_MIX_DEPTH(15) SOPHIA_MIX_DEPTH(16)
#undef SOPHIA_MIX_DEPTH
#undef SOPHIA_MIX_CASE
    default:
      return set_error(SOPHIA_ERR_INVALID, "attn_res_mix: no kernel for depth %d", n_blocks + 1);
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
  SOPHIA_REQUIRE(rows <= 0x7fffffff, "situ_glu: too many rows");
  if (rows == 0) return SOPHIA_OK;
  const int blocks_per_row = (hidden / 8 + 255) / 256;
  const int64_t blocks = rows * blocks_per_row;
  SOPHIA_REQUIRE(blocks <= 0x7fffffff, "situ_glu: too many rows");
  const hipStream_t st = static_cast<hipStream_t>(stream);
  const dim3 grid(static_cast<unsigned>(blocks)), block(256);
  const float rcg = 1.0f / gate_softcap, rcu = 1.0f / up_softcap, scale = gate_softcap * up_softcap;
  const bool bf = dtype == SOPHIA_DTYPE_BF16, cap4 = gate_softcap == 4.0f;
  if (bf && cap4)
    hipLaunchKernelGGL((situ_glu_kernel<true, true>), grid, block, 0, st, gate_up, gate_up_stride, hidden_out,
                       out_stride, hidden, blocks_per_row, rcg, rcu, scale);
  else if (bf)
    hipLaunchKernelGGL((situ_glu_kernel<true, false>), grid, block, 0, st, gate_up, gate_up_stride, hidden_out,
                       out_stride, hidden, blocks_per_row, rcg, rcu, scale);
  else if (cap4)
    hipLaunchKernelGGL((situ_glu_kernel<false, true>), grid, block, 0, st, gate_up, gate_up_stride, hidden_out,
                       out_stride, hidden, blocks_per_row, rcg, rcu, scale);
  else
    hipLaunchKernelGGL((situ_glu_kernel<false, false>), grid, block, 0, st, gate_up, gate_up_stride, hidden_out,
                       out_stride, hidden, blocks_per_row, rcg, rcu, scale);
  return check_launch("situ_glu");
}

extern "C" int sophia_gated_head_norm(const void *o, int64_t o_stride, int o_dtype, const void *gate,
                                      int64_t gate_stride, const float *norm_weight, float eps, void *out,
                                      int64_t out_stride, int64_t rows, int heads, int head_dim, int dtype,
                                      void *stream) {
  SOPHIA_REQUIRE((dtype == SOPHIA_DTYPE_F32 || dtype == SOPHIA_DTYPE_BF16) &&
                     (o_dtype == SOPHIA_DTYPE_F32 || o_dtype == SOPHIA_DTYPE_BF16),
                 "gated_head_norm: dtype not supported");
  SOPHIA_REQUIRE(o_dtype == dtype || o_dtype == SOPHIA_DTYPE_F32, "gated_head_norm: o may be fp32 or the gate's dtype");
  SOPHIA_REQUIRE(head_dim >= 8 && head_dim <= 512 && (head_dim & (head_dim - 1)) == 0,
                 "gated_head_norm: head_dim must be a power of two in [8, 512]");
  SOPHIA_REQUIRE(heads > 0 && rows >= 0 && static_cast<int64_t>(heads) * head_dim <= (1 << 24),
                 "gated_head_norm: bad heads / rows");
  const int64_t width = static_cast<int64_t>(heads) * head_dim;
  SOPHIA_REQUIRE(o_stride % 8 == 0 && gate_stride % 8 == 0 && out_stride % 8 == 0 && o_stride >= width &&
                     gate_stride >= width && out_stride >= width,
                 "gated_head_norm: strides must be multiples of 8 elements and cover a row");
  SOPHIA_REQUIRE(rows == 0 || (o && gate && out), "gated_head_norm: NULL pointer");
  SOPHIA_REQUIRE(aligned16(o) && aligned16(gate) && aligned16(out) && aligned16(norm_weight),
                 "gated_head_norm: pointers must be 16-byte aligned");
  SOPHIA_REQUIRE(rows <= 0x7fffffff, "gated_head_norm: too many rows");
  if (rows == 0) return SOPHIA_OK;
  const int blocks_per_row = static_cast<int>((width / 8 + 255) / 256);
  const int64_t blocks = rows * blocks_per_row;
  SOPHIA_REQUIRE(blocks <= 0x7fffffff, "gated_head_norm: too many rows");
  GateArgs a{o, o_stride, o_dtype, gate, gate_stride, norm_weight, eps, out, out_stride, static_cast<int>(width),
             head_dim, blocks_per_row, dtype};
  hipLaunchKernelGGL(gated_head_norm_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), a);
  return check_launch("gated_head_norm");
}

extern "C" int sophia_mla_latent_norms(void *q_lat, int64_t q_stride, void *kv_lat, int64_t kv_stride, int64_t rows,
                                       int q_rank, int kv_rank, int dtype, const float *q_norm_weight, float q_eps,
                                       const float *kv_norm_weight, float kv_eps, float *latent_cache, int n_slots,
                                       int max_len, int64_t n_prefill_rows, const int32_t *prefill_seq_slots,
                                       int prefill_seq_len, const int64_t *prefill_row_slots,
                                       const int64_t *prefill_row_pos, const int32_t *decode_slots,
                                       const int64_t *decode_pos, void *stream) {
  SOPHIA_REQUIRE(dtype == SOPHIA_DTYPE_F32 || dtype == SOPHIA_DTYPE_BF16, "mla_latent_norms: dtype not supported");
  SOPHIA_REQUIRE(q_rank > 0 && kv_rank > 0 && q_rank % 8 == 0 && kv_rank % 8 == 0 && q_rank + kv_rank <= 512,
                 "mla_latent_norms: ranks must be positive multiples of 8 with q_rank + kv_rank <= 512");
  SOPHIA_REQUIRE(rows >= 0 && rows <= 0x7fffffff && n_prefill_rows >= 0 && n_prefill_rows <= rows,
                 "mla_latent_norms: bad rows / n_prefill_rows");
  SOPHIA_REQUIRE(q_stride % 8 == 0 && kv_stride % 8 == 0 && q_stride >= q_rank && kv_stride >= kv_rank,
                 "mla_latent_norms: strides must be multiples of 8 elements and cover a row");
  SOPHIA_REQUIRE(rows == 0 || (q_lat && kv_lat && q_norm_weight && kv_norm_weight),
                 "mla_latent_norms: NULL pointer");
  SOPHIA_REQUIRE(aligned16(q_lat) && aligned16(kv_lat) && aligned16(q_norm_weight) && aligned16(kv_norm_weight) &&
                     aligned16(latent_cache),
                 "mla_latent_norms: pointers must be 16-byte aligned");
  if (latent_cache) {
    SOPHIA_REQUIRE(n_slots >= 0 && max_len >= 0, "mla_latent_norms: bad cache shape");
    SOPHIA_REQUIRE(n_prefill_rows == 0 || (prefill_seq_slots ? prefill_seq_len > 0
                                                              : (prefill_row_slots && prefill_row_pos)),
                   "mla_latent_norms: prefill rows need their slots and positions");
    SOPHIA_REQUIRE(n_prefill_rows == rows || (decode_slots && decode_pos),
                   "mla_latent_norms: decode rows need their slots and positions");
  }
  if (rows == 0) return SOPHIA_OK;
  MlaNormArgs a{q_lat, q_stride, kv_lat, kv_stride, q_rank, kv_rank, static_cast<int>(rows), q_norm_weight,
                kv_norm_weight, q_eps, kv_eps, latent_cache, n_slots, max_len, static_cast<int>(n_prefill_rows),
                prefill_seq_slots, prefill_seq_len, prefill_row_slots, prefill_row_pos, decode_slots, decode_pos};
  const dim3 grid(static_cast<unsigned>((rows + 3) / 4));
  if (dtype == SOPHIA_DTYPE_BF16)
    hipLaunchKernelGGL(mla_latent_norm_kernel<true>, grid, dim3(256), 0, static_cast<hipStream_t>(stream), a);
  else
    hipLaunchKernelGGL(mla_latent_norm_kernel<false>, grid, dim3(256), 0, static_cast<hipStream_t>(stream), a);
  return check_launch("mla_latent_norms");
}

extern "C" size_t sophia_mla_decode_workspace_size(int64_t rows, int rank, int splits) {
  if (rows < 0 || rank <= 0 || splits < 1) return 0;
  return splits > 1 ? static_cast<size_t>(rows) * splits * 16 * (rank + 2) * sizeof(float) : 0;
}

extern "C" int sophia_mla_decode_attn(const void *qa, int64_t qa_stride, int qa_dtype, const float *latent,
                                      int64_t slot_stride, int n_slots, int max_seq, const int32_t *slots,
                                      const int64_t *pos, float scale, void *out, int64_t out_stride,
                                      int out_dtype, int64_t rows, int heads, int rank, int splits,
                                      void *workspace, size_t workspace_bytes, void *stream) {
  SOPHIA_REQUIRE((qa_dtype == SOPHIA_DTYPE_F32 || qa_dtype == SOPHIA_DTYPE_BF16) &&
                     (out_dtype == SOPHIA_DTYPE_F32 || out_dtype == SOPHIA_DTYPE_BF16),
                 "mla_decode_attn: dtype not supported");
  SOPHIA_REQUIRE(rank == 32 || rank == 64 || rank == 128 || rank == 256,
                 "mla_decode_attn: rank %d not supported (32, 64, 128 or 256)", rank);
  SOPHIA_REQUIRE(heads >= 1 && heads <= 16, "mla_decode_attn: heads must be in [1, 16]");
  SOPHIA_REQUIRE(rows >= 0 && rows <= 0x7fffffff && splits >= 1 && splits <= 65535,
                 "mla_decode_attn: bad rows / splits");
  SOPHIA_REQUIRE(n_slots >= 0 && max_seq >= 0 && slot_stride >= static_cast<int64_t>(max_seq) * rank,
                 "mla_decode_attn: slot stride smaller than a slot");
  SOPHIA_REQUIRE(qa_stride >= static_cast<int64_t>(heads) * rank && out_stride >= static_cast<int64_t>(heads) * rank &&
                     qa_stride % 8 == 0 && slot_stride % 8 == 0,
                 "mla_decode_attn: bad strides");
  SOPHIA_REQUIRE(rows == 0 || (qa && latent && slots && pos && out), "mla_decode_attn: NULL pointer");
  SOPHIA_REQUIRE(aligned16(qa) && aligned16(latent), "mla_decode_attn: qa and latent must be 16-byte aligned");
  SOPHIA_REQUIRE(splits == 1 || (workspace && workspace_bytes >= sophia_mla_decode_workspace_size(rows, rank, splits)),
                 "mla_decode_attn: workspace too small");
  if (rows == 0) return SOPHIA_OK;
  MlaArgs a{qa, qa_stride, qa_dtype, latent, slot_stride, max_seq, n_slots, slots, pos, scale,
            out, out_stride, out_dtype, static_cast<float *>(workspace), heads, splits};
  const hipStream_t st = static_cast<hipStream_t>(stream);
  const dim3 grid(static_cast<unsigned>(rows), static_cast<unsigned>(splits));
  switch (rank) {
#define SOPHIA_MLA_CASE(r)                                                                         \
  case r:                                                                                          \
    hipLaunchKernelGGL(mla_decode_kernel<r>, grid, dim3(256), 0, st, a);                           \
    if (splits > 1) hipLaunchKernelGGL(mla_decode_merge_kernel<r>, dim3(static_cast<unsigned>(rows)), \
                                       dim3(256), 0, st, a);                                       \
    break;
    SOPHIA_MLA_CASE(32) SOPHIA_MLA_CASE(64) SOPHIA_MLA_CASE(128) SOPHIA_MLA_CASE(256)
#undef SOPHIA_MLA_CASE
  }
  return check_launch("mla_decode_attn");
}

extern "C" int sophia_causal_attention(const void *q, int64_t q_stride, const void *k, int64_t k_stride,
                                       const void *v, int64_t v_stride, void *out, int64_t out_stride,
                                       const int32_t *cu_seqlens, const int32_t *cu_seqlens_k, int n_seqs,
                                       int64_t total, int64_t total_k, int max_len, int heads, int head_dim,
                                       float scale, int dtype, void *stream) {
  SOPHIA_REQUIRE(dtype == SOPHIA_DTYPE_BF16, "causal_attention: bf16 only");
  SOPHIA_REQUIRE(head_dim == kFaD, "causal_attention: head_dim must be %d", kFaD);
  SOPHIA_REQUIRE(heads >= 1 && heads <= 65535 && n_seqs >= 0 && n_seqs <= 65535 && total >= 0 && max_len >= 0,
                 "causal_attention: bad heads / sequences");
  const int64_t width = static_cast<int64_t>(heads) * head_dim;
  SOPHIA_REQUIRE(q_stride >= width && k_stride >= width && v_stride >= width && out_stride >= width &&
                     q_stride % 8 == 0 && k_stride % 8 == 0 && v_stride % 8 == 0 && out_stride % 4 == 0,
                 "causal_attention: bad strides");
  SOPHIA_REQUIRE(n_seqs == 0 || total == 0 || (q && k && v && out && cu_seqlens), "causal_attention: NULL pointer");
  SOPHIA_REQUIRE(!cu_seqlens_k || total_k >= 0, "causal_attention: bad total_k");
  SOPHIA_REQUIRE(aligned16(q) && aligned16(k) && aligned16(v) && (reinterpret_cast<uintptr_t>(out) & 7) == 0,
                 "causal_attention: q, k, v must be 16-byte and out 8-byte aligned");
  if (n_seqs == 0 || total == 0 || max_len == 0) return SOPHIA_OK;
  FaArgs a{static_cast<const uint16_t *>(q), static_cast<const uint16_t *>(k), static_cast<const uint16_t *>(v),
           q_stride, k_stride, v_stride, static_cast<uint16_t *>(out), out_stride, cu_seqlens, cu_seqlens_k,
           n_seqs, total, cu_seqlens_k ? total_k : total, (max_len + kFaQ - 1) / kFaQ, heads,
           scale * 1.44269504088896341f};
  const int64_t pair_groups = (static_cast<int64_t>(heads) * n_seqs + 7) / 8;
  const int64_t blocks = pair_groups * 8 * a.q_blocks;
  SOPHIA_REQUIRE(blocks <= 0x7fffffff, "causal_attention: grid too large");
  hipLaunchKernelGGL(causal_attn_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), a);
  return check_launch("causal_attention");
}

extern "C" size_t sophia_gated_head_norm_bwd_workspace_size(int64_t rows, int heads, int head_dim) {
  if (rows < 0 || heads <= 0 || head_dim <= 0) return 0;
  const int64_t width = static_cast<int64_t>(heads) * head_dim;
  const int64_t blocks = ((rows + kGnbRows - 1) / kGnbRows) * ((width / 8 + 255) / 256);
  return static_cast<size_t>(blocks > 0 ? blocks : 1) * head_dim * sizeof(float);
}

extern "C" int sophia_gated_head_norm_bwd(const void *d_out, int64_t d_out_stride, const void *o, int64_t o_stride,
                                          int o_dtype, const void *gate, int64_t gate_stride,
                                          const float *norm_weight, float eps, void *d_o, int64_t d_o_stride,
                                          void *d_gate, int64_t d_gate_stride, float *d_norm_weight, int64_t rows,
                                          int heads, int head_dim, int dtype, void *workspace,
                                          size_t workspace_bytes, void *stream) {
  SOPHIA_REQUIRE((dtype == SOPHIA_DTYPE_F32 || dtype == SOPHIA_DTYPE_BF16) &&
                     (o_dtype == SOPHIA_DTYPE_F32 || o_dtype == SOPHIA_DTYPE_BF16),
                 "gated_head_norm_bwd: dtype not supported");
  SOPHIA_REQUIRE(o_dtype == dtype || o_dtype == SOPHIA_DTYPE_F32,
                 "gated_head_norm_bwd: o may be fp32 or the gate's dtype");
  SOPHIA_REQUIRE(head_dim >= 8 && head_dim <= 256 && (head_dim & (head_dim - 1)) == 0,
                 "gated_head_norm_bwd: head_dim must be a power of two in [8, 256]");
  SOPHIA_REQUIRE(heads > 0 && rows >= 0 && rows <= 0x7fffffff && static_cast<int64_t>(heads) * head_dim <= (1 << 24),
                 "gated_head_norm_bwd: bad heads / rows");
  const int64_t width = static_cast<int64_t>(heads) * head_dim;
  SOPHIA_REQUIRE(d_out_stride % 8 == 0 && o_stride % 8 == 0 && gate_stride % 8 == 0 && d_o_stride % 8 == 0 &&
                     d_gate_stride % 8 == 0 && d_out_stride >= width && o_stride >= width &&
                     gate_stride >= width && d_o_stride >= width && d_gate_stride >= width,
                 "gated_head_norm_bwd: strides must be multiples of 8 elements and cover a row");
  SOPHIA_REQUIRE(rows == 0 || (d_out && o && gate && d_o && d_gate), "gated_head_norm_bwd: NULL pointer");
  SOPHIA_REQUIRE(norm_weight == nullptr || (d_norm_weight && workspace),
                 "gated_head_norm_bwd: the norm weight needs d_norm_weight and a workspace");
  SOPHIA_REQUIRE(aligned16(d_out) && aligned16(o) && aligned16(gate) && aligned16(d_o) && aligned16(d_gate) &&
                     aligned16(norm_weight),
                 "gated_head_norm_bwd: pointers must be 16-byte aligned");
  const int blocks_per_row = static_cast<int>((width / 8 + 255) / 256);
  const int64_t blocks = ((rows + kGnbRows - 1) / kGnbRows) * blocks_per_row;
  SOPHIA_REQUIRE(blocks <= 0x7fffffff, "gated_head_norm_bwd: too many rows");
  if (norm_weight) {
    const size_t need = sophia_gated_head_norm_bwd_workspace_size(rows, heads, head_dim);
    if (workspace_bytes < need)
      return set_error(SOPHIA_ERR_WORKSPACE, "gated_head_norm_bwd: workspace %zu bytes < required %zu",
                       workspace_bytes, need);
  }
  GateBwdArgs a{d_out, d_out_stride, o, o_stride, o_dtype, gate, gate_stride, norm_weight, eps, d_o, d_o_stride,
                d_gate, d_gate_stride, static_cast<float *>(workspace), d_norm_weight, static_cast<int>(rows),
                static_cast<int>(width), head_dim, blocks_per_row, static_cast<int>(blocks), dtype};
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (blocks > 0) {
    hipLaunchKernelGGL(gated_head_norm_bwd_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, st, a);
    if (const int rc = check_launch("gated_head_norm_bwd")) return rc;
  }
  if (norm_weight) {
    hipLaunchKernelGGL(gated_head_norm_dw_reduce_kernel, dim3((head_dim + 255) / 256), dim3(256), 0, st, a);
    return check_launch("gated_head_norm_dw_reduce");
  }
  return SOPHIA_OK;
}
