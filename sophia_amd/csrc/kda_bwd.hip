// KDA backward over a packed ragged batch (training), gfx950.
//
// Gradients of the prefill (the chunk forward with a zero or given initial
// state) with respect to q, k, v, g, beta, the initial state, A_log and
// dt_bias.  Replaces FlashKDA's chunk_kda_train_bwd together with the
// l2norm_bwd and fused_beta_sigmoid_bwd calls after it, as FlashKDAFunction.
// backward makes them (ml/training/pretrain/engine/sm120_concurrent_ffn.py:
// 301-373, the call at 320).
//
// Per token t of a sequence (q^ = q/|q| * scale, k^ = k/|k|, alpha = e^g):
//   S~ = Diag(alpha) S_{t-1},  p = k^T S~,  u = beta (v - p),
//   S_t = S~ + k^ u^T,         o_t = S_t^T q^
// and in reverse, with dS the gradient of S_t (dS_T = dht):
//   dS += q^ do^T;  dq^ = S_t do;  du = dS^T k^;  dv = beta du;
//   dbeta = du . (v - p);  dp = -beta du;  dk^ = dS u + S~ dp;
//   dS~ = dS + k^ dp^T;  dalpha = rowsum(dS~ o S_{t-1});  dS_{t-1} = Diag(alpha) dS~.
//
// Two forms.  The default, the chunk form, is kda_chunk.hip's chunk_bwd_run
// (backward records, forward-state and reverse chunk scans, per-chunk
// gradients on MFMA, the norms', gate's and sigmoid's backward inside the
// last kernel) followed by the gate-parameter sums below.  The recurrent
// form (SOPHIA_KDA_BWD_RECURRENT) runs the per-token recurrence in fp32:
//
// Kernels of the recurrent form:
//  * kda_bwd_prep_kernel, one work-group of 128 threads per (token, head):
//    q^, k^, the decay alpha = e^g (gate applied) and beta (sigmoid applied),
//    fp32.
//  * kda_bwd_chain_kernel, one work-group of 512 threads per (sequence, head,
//    32-column value slice): the value columns of the state evolve
//    independently, so each slice runs the recurrence alone.  It first runs
//    the sequence forward and keeps the state at every 8-token piece start in
//    the workspace (64 KiB per piece and head); then it takes the pieces in
//    reverse, recomputes each piece's 8 states in registers from its
//    checkpoint and runs the reverse steps: two passes over the tokens plus
//    the recompute.  Every piece it walks is staged in LDS by the whole
//    work-group, the next piece's loads in flight while the current one is
//    processed.  Sums over value columns (dq^, dk^, dalpha, and dbeta in the
//    same column reduction) leave as per-slice partials.
//  * kda_bwd_post_kernel, one work-group of 128 threads per (token, head):
//    sums the partials and applies the backward of the l2 norms, of the gate
//    g = lb sigmoid(e^A_log (z + dt_bias)) and of the beta sigmoid.
//  * kda_bwd_gate_partial_kernel / kda_bwd_gate_final_kernel (both forms):
//    dA_log and ddt_bias, sums over tokens of dz (z + dt_bias) and dz, in a
//    fixed order.
//
// Thread t of the chain kernel owns value column j = t % 32 of its slice and
// state rows 8 (t / 32) .. +7.  A sum over the 128 rows (k^T X for a column)
// is 8 local terms, a xor-32 shuffle and 8 wavefront partials through LDS (one
// barrier); a sum over the 32 columns (X z for a row) is a butterfly inside
// each half-wavefront that leaves the sum of value i in lane i.
#include <mutex>

#include "common.hpp"
#include "kda_chunk_bwd.hpp"

namespace sophia {
namespace {

constexpr int kD = 128;
constexpr int kSub = 8;          // checkpoint interval: one piece of tokens
constexpr int kNV = 32;          // value columns per work-group
constexpr int kSlices = kD / kNV;
constexpr int kChainThreads = 512;
constexpr int kRows = kD / (kChainThreads / kNV);   // state rows per thread: 8
constexpr int kGateParts = 64;   // token partitions of the dA_log / ddt_bias sums
constexpr int kMaxDevices = 64;
constexpr size_t kChainLdsFloats = 2 * 8 * kNV;

struct BwdArgs {
  // inputs
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
  const float *h0;        // [n_seqs, H, 128, 128] or NULL
  const void *dout;       // [total, H, 128] rows of do_stride elements
  int64_t do_stride;
  int do_dtype;
  const float *dht;       // [n_seqs, H, 128, 128] or NULL
  // outputs: dq, dk, dv of element type grad_dtype, the others fp32
  void *dq, *dk, *dv;
  int grad_dtype;
  float *dg, *dbeta, *dh0, *dA_log, *ddt_bias;
  // workspace
  float *qh, *kh, *gl, *bt;        // prepared q^, k^, alpha = e^g, beta
  float *ckpt;                     // [pieces, H, 128, 128] states at every 8-token piece start
  float *dqh, *dkh, *dal;          // [kSlices, total, H, 128] partial sums
  float *dbp;                      // [kSlices, total, H] dbeta summed over a slice's columns
  float *pv;                       // [total, H, 128] p = k^T S~ of every token (forward walk)
  float *gpb, *gpa;                // [kGateParts, H, 128] partial ddt_bias / dA_log
};

// ---- prep ---------------------------------------------------------------------
__global__ __launch_bounds__(kD) void kda_bwd_prep_kernel(BwdArgs a) {
  const int64_t tok = blockIdx.x;
  const int h = blockIdx.y;
  const int c = threadIdx.x;
  __shared__ float s_red[2][2];
  const int64_t row = tok * a.qkv_stride + static_cast<int64_t>(h) * kD + c;
  const float qv = load_elem(a.q, row, a.qkv_dtype);
  const float kv = load_elem(a.k, row, a.qkv_dtype);
  float z = load_elem(a.g, tok * a.g_stride + static_cast<int64_t>(h) * kD + c, a.g_dtype);
  float b = load_elem(a.beta, tok * a.beta_stride + h, a.beta_dtype);
  const float sq = wave_sum(qv * qv), sk = wave_sum(kv * kv);
  if ((c & 63) == 0) {
    s_red[c >> 6][0] = sq;
    s_red[c >> 6][1] = sk;
  }
  __syncthreads();
  float qs = a.scale, ks = 1.f;
  if (a.flags & SOPHIA_KDA_QK_L2NORM) {
    qs /= fmaxf(sqrtf(s_red[0][0] + s_red[1][0]), 1e-12f);
    ks /= fmaxf(sqrtf(s_red[0][1] + s_red[1][1]), 1e-12f);
  }
  if (a.flags & SOPHIA_KDA_GATE_IN_KERNEL)
    z = a.lb / (1.f + expf(-expf(a.A_log[h]) * (z + a.dt_bias[h * kD + c])));
  const int64_t o = (tok * a.num_heads + h) * kD + c;
  a.qh[o] = qv * qs;
  a.kh[o] = kv * ks;
  a.gl[o] = expf(z);
  if (c == 0) {
    if (a.flags & SOPHIA_KDA_BETA_SIGMOID) b = 1.f / (1.f + expf(-b));
    a.bt[tok * a.num_heads + h] = b;
  }
}

// ---- chain --------------------------------------------------------------------
// The inputs of one 8-token piece, staged in LDS for the whole work-group
// (rows of q^, k^, alpha; the slice's 32 columns of v and of do; beta).
struct Piece {
  float q[kSub][kD], k[kSub][kD], al[kSub][kD];
  float v[kSub][kNV], dout[kSub][kNV], p[kSub][kNV];
  float bt[kSub];
};

constexpr size_t kChainLds = kChainLdsFloats * sizeof(float) + 2 * sizeof(Piece);

struct ChainCtx {
  const BwdArgs *a;
  int h, col, j, rg, lane, wave;
  float *s_kred;    // [2][8 waves][32]
};

// DPP within 16-lane rows (the exchanges across rows are lane_xor16 /
// lane_xor32, gfx950's row swaps).
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}

// Sum over the 128 state rows of x (one partial per thread, over its 8 rows)
// for the thread's column.  Consecutive calls alternate between two LDS
// buffers, so a buffer is rewritten only after every thread has passed the
// barrier of the call in between (and so has read it).
__device__ __forceinline__ float row_sum(const ChainCtx &c, float x, int &kb) {
  x += lane_xor32(x);
  float *buf = c.s_kred + kb * 8 * kNV;
  kb ^= 1;
  if (c.lane < kNV) buf[c.wave * kNV + c.j] = x;
  lds_barrier();
  float s = 0.f;
#pragma unroll
  for (int w = 0; w < 8; ++w) s += buf[w * kNV + c.j];
  return s;
}

// The inputs of one token for the thread's rows and column.
struct TokenIn {
  f4 q[kRows / 4], k[kRows / 4], al[kRows / 4];
  float v, bt, dout;
};

__device__ __forceinline__ void token_from(const ChainCtx &c, const Piece &pc, int t, TokenIn &in) {
#pragma unroll
  for (int i = 0; i < kRows / 4; ++i) {
    in.q[i] = *reinterpret_cast<const f4 *>(&pc.q[t][c.rg * kRows + 4 * i]);
    in.k[i] = *reinterpret_cast<const f4 *>(&pc.k[t][c.rg * kRows + 4 * i]);
    in.al[i] = *reinterpret_cast<const f4 *>(&pc.al[t][c.rg * kRows + 4 * i]);
  }
  in.v = pc.v[t][c.j];
  in.dout = pc.dout[t][c.j];
  in.bt = pc.bt[t];
}

__device__ __forceinline__ float tq(const TokenIn &in, int i) { return in.q[i >> 2][i & 3]; }
__device__ __forceinline__ float tk(const TokenIn &in, int i) { return in.k[i >> 2][i & 3]; }
__device__ __forceinline__ float talpha(const TokenIn &in, int i) { return in.al[i >> 2][i & 3]; }

// S <- S_t from S_{t-1}; returns p = k^T S~ of the thread's column.
__device__ __forceinline__ float fwd_step(const ChainCtx &c, const TokenIn &in, float (&S)[kRows], int &kb) {
  float part = 0.f;
#pragma unroll
  for (int i = 0; i < kRows; ++i) {
    S[i] *= talpha(in, i);
    part = fmaf(tk(in, i), S[i], part);
  }
  const float p = row_sum(c, part, kb);
  const float u = in.bt * (in.v - p);
#pragma unroll
  for (int i = 0; i < kRows; ++i) S[i] = fmaf(tk(in, i), u, S[i]);
  return p;
}

// One butterfly stage: of x[0 .. 2N) keep the half selected by lane bit m and
// add the partner lane's copy of that half.  The partner differs in bit m
// and in lower bits only: lane ^ 16 (row swap), the mirrored lane of the
// 16-lane row (lane ^ 15, DPP row_mirror), of the 8-lane half-row (lane ^ 7,
// row_half_mirror), lane ^ 2 and lane ^ 1 (quad_perm).  Partners hold the
// same half before the stage, so the halves exchange cleanly, and the
// partner masks 16, 15, 7, 2, 1 together reach all 32 lanes.
template <int N, int M>
__device__ __forceinline__ void fold(const float (&x)[2 * N], float (&y)[N], int l) {
  const bool up = (l & M) != 0;
#pragma unroll
  for (int i = 0; i < N; ++i) {
    const float keep = up ? x[N + i] : x[i], send = up ? x[i] : x[N + i];
    float got;
    if constexpr (M == 16) got = lane_xor16(send);
    else if constexpr (M == 8) got = dpp<0x140>(send);     // row_mirror
    else if constexpr (M == 4) got = dpp<0x141>(send);     // row_half_mirror
    else if constexpr (M == 2) got = dpp<0x4E>(send);      // quad_perm 2,3,0,1
    else got = dpp<0xB1>(send);                            // quad_perm 1,0,3,2
    y[i] = keep + got;
  }
}

// Sum over the 32 lanes of a half-wavefront: on return lane i holds the sum
// over those lanes of x[i].
__device__ __forceinline__ float col_sum32(const float (&x)[32], int l) {
  float y16[16], y8[8], y4[4], y2[2], y1[1];
  fold<16, 16>(x, y16, l);
  fold<8, 8>(y16, y8, l);
  fold<4, 4>(y8, y4, l);
  fold<2, 2>(y4, y2, l);
  fold<1, 1>(y2, y1, l);
  return y1[0];
}

// The loads of one piece (tokens [tok0, tok0 + m)) into the LDS piece at
// `dst` (byte address of its q field): the rows of q^, k^ and alpha go
// straight to LDS, 1 KiB (two token rows) per wavefront instruction, lane l
// writing bytes 16 l .. 16 l + 15 of its block; v, do and beta come into
// registers and are stored by piece_store.  Rows past m re-read row m - 1.
struct PieceRegs {
  float s[2];
};

// with_p: also the slice's p values of the piece (written by the forward walk).
__device__ __forceinline__ void piece_load(const BwdArgs &a, int h, int col0, int64_t tok0, int m, uint8_t *dst,
                                           bool with_p, PieceRegs &r) {
  const int t = threadIdx.x;
  const int w = t >> 6, l = t & 63;
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int blk = w + 8 * u;             // 12 blocks: 3 arrays x 4 token pairs
    if (blk < 3 * kSub / 2) {
      const int arr = blk / (kSub / 2), pair = blk % (kSub / 2);
      const int tok = min(2 * pair + (l >> 5), m - 1);
      const float *src = (arr == 0 ? a.qh : (arr == 1 ? a.kh : a.gl)) +
                         ((tok0 + tok) * a.num_heads + h) * kD + 4 * (l & 31);
      __builtin_amdgcn_global_load_lds(src, dst + arr * (kSub * kD * 4) + pair * 1024, 16, 0, 0);
    }
  }
  const int which = t >> 8, rem = t & 255, tok = rem >> 5, cj = rem & 31;
  float val = 0.f;
  if (tok < m) {
    if (which == 0)
      val = load_elem(a.v, (tok0 + tok) * a.qkv_stride + static_cast<int64_t>(h) * kD + col0 + cj, a.qkv_dtype);
    else
      val = load_elem(a.dout, (tok0 + tok) * a.do_stride + static_cast<int64_t>(h) * kD + col0 + cj, a.do_dtype);
  }
  r.s[0] = val;
  // threads 0 .. 255: p (8 tokens x 32 columns); 256 .. 263: beta
  float v1 = 0.f;
  if (which == 0) {
    if (with_p && tok < m) v1 = a.pv[((tok0 + tok) * a.num_heads + h) * kD + col0 + cj];
  } else if (rem < kSub && rem < m) {
    v1 = a.bt[(tok0 + rem) * a.num_heads + h];
  }
  r.s[1] = v1;
}

__device__ __forceinline__ void piece_store(Piece &pc, const PieceRegs &r) {
  const int t = threadIdx.x;
  const int which = t >> 8, rem = t & 255, tok = rem >> 5, cj = rem & 31;
  (which == 0 ? pc.v : pc.dout)[tok][cj] = r.s[0];
  if (which == 0)
    pc.p[tok][cj] = r.s[1];
  else if (rem < kSub)
    pc.bt[rem] = r.s[1];
}

__global__ __launch_bounds__(kChainThreads) void kda_bwd_chain_kernel(BwdArgs a) {
  extern __shared__ __attribute__((aligned(16))) float smem[];
  float *s_kred = smem;                                              // [2][8][32]
  Piece *s_pc = reinterpret_cast<Piece *>(s_kred + 2 * 8 * kNV);     // [2]
  uint8_t *s_pc_bytes = reinterpret_cast<uint8_t *>(smem) + kChainLdsFloats * sizeof(float);

  const int s = blockIdx.x / (a.num_heads * kSlices);
  const int rem = blockIdx.x % (a.num_heads * kSlices);
  const int h = rem / kSlices;
  const int slice = rem % kSlices;
  if (s >= a.n_seqs) return;
  ChainCtx c;
  c.a = &a;
  c.h = h;
  c.j = threadIdx.x % kNV;
  c.col = slice * kNV + c.j;
  c.rg = threadIdx.x / kNV;
  c.lane = threadIdx.x & 63;
  c.wave = threadIdx.x >> 6;
  c.s_kred = s_kred;
  const int l32 = threadIdx.x & 31;
  const int r0 = c.rg * kRows;
  const int col0 = slice * kNV;
  const int64_t seq_a = iclamp64(a.cu[s], 0, a.total);
  const int64_t seq_b = iclamp64(a.cu[s + 1], seq_a, a.total);
  const int len = static_cast<int>(seq_b - seq_a);
  const int np = (len + kSub - 1) / kSub;   // 8-token pieces
  // Checkpoint slots of this sequence: seq_a / 8 + s + piece.  For ordered
  // offsets the sequences' slots do not overlap, and for any offsets they
  // stay below total / 8 + n_seqs.
  const int64_t ck0 = seq_a / kSub + s;
  const int64_t state_off = (static_cast<int64_t>(s) * a.num_heads + h) * kD * kD;
  int kb = 0;

  float S[kRows], dS[kRows];
#pragma unroll
  for (int i = 0; i < kRows; ++i) {
    S[i] = a.h0 ? a.h0[state_off + static_cast<int64_t>(r0 + i) * kD + c.col] : 0.f;
    dS[i] = a.dht ? a.dht[state_off + static_cast<int64_t>(r0 + i) * kD + c.col] : 0.f;
  }
  // The state before piece p (rows r0.., column col of this thread): written
  // by the forward walk, read back by the same thread in the reverse walk.
  const auto ckpt = [&](int p, int i) -> float & {
    return a.ckpt[((ck0 + p) * a.num_heads + h) * kD * kD + static_cast<int64_t>(r0 + i) * kD + c.col];
  };
  const auto count_of = [&](int p) { return min(kSub, len - p * kSub); };

  if (np > 0) {
    // Walk: pieces 0 .. np - 1 forward (v = p), then np - 1 .. 0 in reverse
    // (v = 2 np - 1 - p); each piece's inputs staged in LDS one visit ahead.
    const int nvis = 2 * np;
    const auto piece_of = [&](int vis) { return vis < np ? vis : 2 * np - 1 - vis; };
    int cb = 0;
    {
      PieceRegs r;
      piece_load(a, h, col0, seq_a, count_of(0), s_pc_bytes, false, r);
      piece_store(s_pc[0], r);
    }
    __syncthreads();
    for (int vis = 0; vis < nvis; ++vis) {
      const int p = piece_of(vis);
      const bool more = vis + 1 < nvis;
      // The last forward visit is followed by the reverse visit of the same
      // piece: that piece stays in its buffer, its p values written there.
      const bool same_next = vis == np - 1;
      PieceRegs r;
      if (more && !same_next) {
        const int pn = piece_of(vis + 1);
        piece_load(a, h, col0, seq_a + static_cast<int64_t>(pn) * kSub, count_of(pn),
                   s_pc_bytes + (cb ^ 1) * sizeof(Piece), vis + 1 >= np, r);
      }
      Piece &pc = s_pc[cb];
      const int m = count_of(p);
      if (vis < np) {
#pragma unroll
        for (int i = 0; i < kRows; ++i) ckpt(p, i) = S[i];
        const int64_t p0 = seq_a + static_cast<int64_t>(p) * kSub;
#pragma unroll 1
        for (int t = 0; t < m; ++t) {
          TokenIn in;
          token_from(c, pc, t, in);
          const float pt = fwd_step(c, in, S, kb);
          if (c.rg == 0) {
            a.pv[((p0 + t) * a.num_heads + h) * kD + c.col] = pt;
            pc.p[t][c.j] = pt;
          }
        }
      } else {
        const int64_t p0 = seq_a + static_cast<int64_t>(p) * kSub;
        // Sp[t]: the state before token t of the piece, recomputed from the
        // checkpoint with the p values of the forward walk (so without the
        // cross-row sum: no barrier).
        float Sp[kSub][kRows];
#pragma unroll
        for (int i = 0; i < kRows; ++i) S[i] = ckpt(p, i);
#pragma unroll
        for (int t = 0; t < kSub; ++t) {
          if (t < m) {
            TokenIn in;
            token_from(c, pc, t, in);
            const float u = in.bt * (in.v - pc.p[t][c.j]);
#pragma unroll
            for (int i = 0; i < kRows; ++i) {
              Sp[t][i] = S[i];
              S[i] = fmaf(tk(in, i), u, S[i] * talpha(in, i));
            }
          }
          // one token's LDS reads at a time: hoisting all of them would
          // need more registers than the wavefront has
          __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
        for (int tt = kSub - 1; tt >= 0; --tt) {
          if (tt < m) {
            const int64_t tok = p0 + tt;
            TokenIn cur;
            token_from(c, pc, tt, cur);
            const float dov = cur.dout;
            const float vp = cur.v - pc.p[tt][c.j];
            const float u = cur.bt * vp;
            float x[32];
            float part = 0.f;
#pragma unroll
            for (int i = 0; i < kRows; ++i) {
              dS[i] = fmaf(tq(cur, i), dov, dS[i]);      // dS_t += q^ do^T
              const float st_i = fmaf(tk(cur, i), u, talpha(cur, i) * Sp[tt][i]);   // S_t
              x[i] = st_i * dov;                         // dq^ partial: S_t do
              part = fmaf(tk(cur, i), dS[i], part);
            }
            const float du = row_sum(c, part, kb);       // dS_t^T k^
            const float dp = -cur.bt * du;
#pragma unroll
            for (int i = 0; i < kRows; ++i) {
              const float al = talpha(cur, i);
              const float st = al * Sp[tt][i];                  // S~
              x[kRows + i] = fmaf(dS[i], u, st * dp);           // dk^ partial
              const float dst = fmaf(tk(cur, i), dp, dS[i]);    // dS~
              x[2 * kRows + i] = dst * Sp[tt][i];               // dalpha partial
              dS[i] = al * dst;                                 // dS_{t-1}
            }
            x[3 * kRows] = du * vp;                             // dbeta term of this column
#pragma unroll
            for (int i = 3 * kRows + 1; i < 32; ++i) x[i] = 0.f;
            const float rsum = col_sum32(x, l32);
            if (l32 < 3 * kRows) {
              const int vec = l32 / kRows, row = r0 + (l32 % kRows);
              float *dst = vec == 0 ? a.dqh : (vec == 1 ? a.dkh : a.dal);
              dst[((static_cast<int64_t>(slice) * a.total + tok) * a.num_heads + h) * kD + row] = rsum;
            }
            if (c.rg == 0) {
              store_elem(a.dv, (tok * a.num_heads + h) * kD + c.col, a.grad_dtype, cur.bt * du);
              if (l32 == 3 * kRows) a.dbp[(static_cast<int64_t>(slice) * a.total + tok) * a.num_heads + h] = rsum;
            }
          }
          __builtin_amdgcn_sched_barrier(0);
        }
      }
      if (!more) break;
      if (same_next) {
        __syncthreads();  // this piece's p values are in LDS
      } else {
        piece_store(s_pc[cb ^ 1], r);
        __syncthreads();  // the next piece is in LDS; this one is no longer read
        cb ^= 1;
      }
    }
  }
  if (a.dh0) {
#pragma unroll
    for (int i = 0; i < kRows; ++i) a.dh0[state_off + static_cast<int64_t>(r0 + i) * kD + c.col] = dS[i];
  }
}

// ---- post -----------------------------------------------------------------------
__global__ __launch_bounds__(kD) void kda_bwd_post_kernel(BwdArgs a) {
  const int64_t tok = blockIdx.x;
  const int h = blockIdx.y;
  const int c = threadIdx.x;
  __shared__ float s_red[2][4];
  const int64_t o = (tok * a.num_heads + h) * kD + c;
  float dqh = 0.f, dkh = 0.f, dal = 0.f;
  for (int sl = 0; sl < kSlices; ++sl) {
    const int64_t po = ((static_cast<int64_t>(sl) * a.total + tok) * a.num_heads + h) * kD + c;
    dqh += a.dqh[po];
    dkh += a.dkh[po];
    dal += a.dal[po];
  }
  const int64_t row = tok * a.qkv_stride + static_cast<int64_t>(h) * kD + c;
  const float qv = load_elem(a.q, row, a.qkv_dtype);
  const float kv = load_elem(a.k, row, a.qkv_dtype);
  const bool l2 = (a.flags & SOPHIA_KDA_QK_L2NORM) != 0;
  // With the norm, y = x / n (n = max(|x|, eps)) and dx = (dy - y (y . dy)) / n
  // where |x| >= eps, dx = dy / n where the clamp holds n constant; y . dy is
  // formed as (x . dy) / n, so y is not read back.
  const float dyq = dqh * a.scale;
  const float r0 = wave_sum(qv * dyq), r1 = wave_sum(kv * dkh), r2 = wave_sum(qv * qv),
              r3 = wave_sum(kv * kv);
  if ((c & 63) == 0) {
    s_red[c >> 6][0] = r0;
    s_red[c >> 6][1] = r1;
    s_red[c >> 6][2] = r2;
    s_red[c >> 6][3] = r3;
  }
  __syncthreads();
  float dq = dyq, dk = dkh;
  if (l2) {
    const float lq = sqrtf(s_red[0][2] + s_red[1][2]), lk = sqrtf(s_red[0][3] + s_red[1][3]);
    const float nq = fmaxf(lq, 1e-12f), nk = fmaxf(lk, 1e-12f);
    const float yq = qv / nq, yk = kv / nk;
    dq = (lq < 1e-12f ? dyq : dyq - yq * ((s_red[0][0] + s_red[1][0]) / nq)) / nq;
    dk = (lk < 1e-12f ? dkh : dkh - yk * ((s_red[0][1] + s_red[1][1]) / nk)) / nk;
  }
  store_elem(a.dq, o, a.grad_dtype, dq);
  store_elem(a.dk, o, a.grad_dtype, dk);
  // alpha = e^g: dg = dalpha alpha; through the gate, dz = dg lb s (1 - s) e^A_log
  float dgv = dal * a.gl[o];
  if (a.flags & SOPHIA_KDA_GATE_IN_KERNEL) {
    const float z = load_elem(a.g, tok * a.g_stride + static_cast<int64_t>(h) * kD + c, a.g_dtype);
    const float ea = expf(a.A_log[h]);
    const float sg = 1.f / (1.f + expf(-ea * (z + a.dt_bias[h * kD + c])));
    dgv = dgv * a.lb * sg * (1.f - sg) * ea;
  }
  a.dg[o] = dgv;
  if (c == 0) {
    float db = 0.f;
    for (int sl = 0; sl < kSlices; ++sl) db += a.dbp[(static_cast<int64_t>(sl) * a.total + tok) * a.num_heads + h];
    if (a.flags & SOPHIA_KDA_BETA_SIGMOID) {
      const float bt = a.bt[tok * a.num_heads + h];
      db *= bt * (1.f - bt);
    }
    a.dbeta[tok * a.num_heads + h] = db;
  }
}

// Token rows [lo, hi) covered by the sequences: cu[0] .. cu[n], clamped into
// [0, total] as every kernel clamps the offsets.
__device__ __forceinline__ void covered_rows(const BwdArgs &a, int64_t &lo, int64_t &hi) {
  lo = iclamp64(a.cu[0], 0, a.total);
  hi = iclamp64(a.cu[a.n_seqs], lo, a.total);
}

// ---- rows outside every sequence ---------------------------------------------------
// A batch whose offsets end before its last row (cu[n] < total, or cu[0] > 0)
// has rows no sequence covers; their gradients are zero (the chunk form zeroes
// them in its state-scan kernel).
constexpr int kZeroBlocks = 64;
__global__ __launch_bounds__(256) void kda_bwd_zero_outside_kernel(BwdArgs a) {
  zero_rows_outside(a.cu, a.n_seqs, a.total, a.num_heads, a.dq, a.dk, a.dv, a.grad_dtype, a.dg, a.dbeta,
                    static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x, static_cast<int64_t>(kZeroBlocks) * 256);
}

// ---- gate parameters ---------------------------------------------------------------
// g = lb sigmoid(e^A_log (z + b)): dA_log = sum dz (z + b), ddt_bias = sum dz,
// over the rows the sequences cover.
__global__ __launch_bounds__(kD) void kda_bwd_gate_partial_kernel(BwdArgs a) {
  const int h = blockIdx.x, part = blockIdx.y, c = threadIdx.x;
  int64_t lo, hi;
  covered_rows(a, lo, hi);
  const int64_t per = (hi - lo + kGateParts - 1) / kGateParts;
  const int64_t t_lo = imin64(lo + static_cast<int64_t>(part) * per, hi);
  const int64_t t_hi = imin64(t_lo + per, hi);
  const float b = a.dt_bias[h * kD + c];
  float sb = 0.f, sa = 0.f;
  for (int64_t tok = t_lo; tok < t_hi; ++tok) {
    const float dz = a.dg[(tok * a.num_heads + h) * kD + c];
    const float z = load_elem(a.g, tok * a.g_stride + static_cast<int64_t>(h) * kD + c, a.g_dtype);
    sb += dz;
    sa = fmaf(dz, z + b, sa);
  }
  const int64_t o = (static_cast<int64_t>(part) * a.num_heads + h) * kD + c;
  a.gpb[o] = sb;
  a.gpa[o] = sa;
}

__global__ __launch_bounds__(kD) void kda_bwd_gate_final_kernel(BwdArgs a) {
  const int h = blockIdx.x, c = threadIdx.x;
  __shared__ float s_red[2];
  float sb = 0.f, sa = 0.f;
  for (int part = 0; part < kGateParts; ++part) {
    const int64_t o = (static_cast<int64_t>(part) * a.num_heads + h) * kD + c;
    sb += a.gpb[o];
    sa += a.gpa[o];
  }
  if (a.ddt_bias) a.ddt_bias[h * kD + c] = sb;
  sa = wave_sum(sa);
  if ((c & 63) == 0) s_red[c >> 6] = sa;
  __syncthreads();
  if (c == 0 && a.dA_log) a.dA_log[h] = s_red[0] + s_red[1];
}

size_t align256(size_t x) { return (x + 255) & ~static_cast<size_t>(255); }

size_t max_pieces(int64_t total_tokens, int n_seqs) {
  return static_cast<size_t>(total_tokens / kSub) + static_cast<size_t>(n_seqs);
}

int ensure_chain_lds() {
  static std::mutex mu;
  static bool done[kMaxDevices] = {};
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return set_error(SOPHIA_ERR_HIP, "kda_chunk_bwd: hipGetDevice: %s", hipGetErrorString(e));
  std::lock_guard<std::mutex> lock(mu);
  if (dev >= 0 && dev < kMaxDevices && done[dev]) return SOPHIA_OK;
  e = hipFuncSetAttribute(reinterpret_cast<const void *>(&kda_bwd_chain_kernel),
                          hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(kChainLds));
  if (e != hipSuccess)
    return set_error(SOPHIA_ERR_HIP, "kda_chunk_bwd: cannot set LDS size: %s", hipGetErrorString(e));
  if (dev >= 0 && dev < kMaxDevices) done[dev] = true;
  return SOPHIA_OK;
}

}  // namespace
}  // namespace sophia

using namespace sophia;

// Workspace: the prepared inputs (recurrent form) and the gate partials (both
// forms), then either form's own part.
namespace {
size_t bwd_common_bytes(size_t tok, int num_heads) {
  return 3 * align256(tok * kD * 4) + align256(tok * 4) + 2 * align256(static_cast<size_t>(kGateParts) * num_heads * kD * 4);
}
size_t bwd_recurrent_bytes(int64_t total_tokens, int n_seqs, int num_heads, size_t tok) {
  return align256(max_pieces(total_tokens, n_seqs) * num_heads * kD * kD * 4) + 3 * align256(kSlices * tok * kD * 4) +
         align256(kSlices * tok * 4) + align256(tok * kD * 4);
}
size_t bwd_chunk_bytes(int64_t total_tokens, int n_seqs, int num_heads, size_t) {
  return align256(chunk_bwd_scratch_bytes(total_tokens, n_seqs, num_heads));
}
}  // namespace

extern "C" size_t sophia_kda_chunk_bwd_workspace_size(int64_t total_tokens, int n_seqs, int num_heads,
                                                      int head_dim) {
  if (total_tokens < 0 || n_seqs <= 0 || num_heads <= 0 || head_dim != kD) return 0;
  const size_t tok = static_cast<size_t>(total_tokens) * num_heads;
  const size_t rec = bwd_recurrent_bytes(total_tokens, n_seqs, num_heads, tok);
  const size_t chk = bwd_chunk_bytes(total_tokens, n_seqs, num_heads, tok);
  return bwd_common_bytes(tok, num_heads) + (rec > chk ? rec : chk);
}

extern "C" int sophia_kda_chunk_bwd(const void *q, const void *k, const void *v, int64_t qkv_row_stride,
                                    int qkv_dtype, const void *g, int64_t g_row_stride, int g_dtype,
                                    const void *beta, int64_t beta_row_stride, int beta_dtype,
                                    const float *A_log, const float *dt_bias, float scale, float lower_bound,
                                    unsigned flags, const int32_t *cu_seqlens, int n_seqs, int64_t total_tokens,
                                    int num_heads, int head_dim, const float *initial_state, const void *d_out,
                                    int64_t d_out_row_stride, int d_out_dtype, const float *d_final_state,
                                    void *dq, void *dk, void *dv, float *dg, float *dbeta,
                                    float *d_initial_state, float *dA_log, float *ddt_bias, void *workspace,
                                    size_t workspace_bytes, void *stream) {
  SOPHIA_REQUIRE(head_dim == kD, "kda_chunk_bwd: head_dim must be 128 (got %d)", head_dim);
  SOPHIA_REQUIRE(n_seqs > 0 && num_heads > 0 && num_heads <= 65535 && total_tokens >= 0 &&
                     total_tokens <= 0x7fffffff,
                 "kda_chunk_bwd: bad n_seqs / num_heads / total_tokens");
  SOPHIA_REQUIRE(qkv_dtype == SOPHIA_DTYPE_F32 || qkv_dtype == SOPHIA_DTYPE_BF16, "kda_chunk_bwd: qkv dtype");
  SOPHIA_REQUIRE(g_dtype == SOPHIA_DTYPE_F32 || g_dtype == SOPHIA_DTYPE_BF16, "kda_chunk_bwd: g dtype");
  SOPHIA_REQUIRE(beta_dtype == SOPHIA_DTYPE_F32 || beta_dtype == SOPHIA_DTYPE_BF16, "kda_chunk_bwd: beta dtype");
  SOPHIA_REQUIRE(d_out_dtype == SOPHIA_DTYPE_F32 || d_out_dtype == SOPHIA_DTYPE_BF16,
                 "kda_chunk_bwd: d_out dtype");
  SOPHIA_REQUIRE(cu_seqlens && workspace &&
                     (total_tokens == 0 || (q && k && v && g && beta && d_out && dq && dk && dv && dg && dbeta)),
                 "kda_chunk_bwd: NULL pointer");
  const bool gate = (flags & SOPHIA_KDA_GATE_IN_KERNEL) != 0;
  SOPHIA_REQUIRE(!gate || (A_log && dt_bias), "kda_chunk_bwd: gate in kernel needs A_log and dt_bias");
  SOPHIA_REQUIRE(gate || (!dA_log && !ddt_bias),
                 "kda_chunk_bwd: dA_log / ddt_bias exist only with the gate in the kernel");
  SOPHIA_REQUIRE(qkv_row_stride >= static_cast<int64_t>(num_heads) * kD &&
                     g_row_stride >= static_cast<int64_t>(num_heads) * kD && beta_row_stride >= num_heads &&
                     d_out_row_stride >= static_cast<int64_t>(num_heads) * kD,
                 "kda_chunk_bwd: row stride smaller than a row");
  SOPHIA_REQUIRE((reinterpret_cast<uintptr_t>(workspace) % 256) == 0,
                 "kda_chunk_bwd: workspace must be 256-byte aligned");
  const int64_t blocks = static_cast<int64_t>(n_seqs) * num_heads * kSlices;
  SOPHIA_REQUIRE(blocks <= 0x7fffffff, "kda_chunk_bwd: grid too large");
  const size_t need = sophia_kda_chunk_bwd_workspace_size(total_tokens, n_seqs, num_heads, head_dim);
  if (workspace_bytes < need)
    return set_error(SOPHIA_ERR_WORKSPACE, "kda_chunk_bwd: workspace %zu bytes < required %zu", workspace_bytes,
                     need);
  const size_t tok = static_cast<size_t>(total_tokens) * num_heads;
  uint8_t *w = static_cast<uint8_t *>(workspace);
  auto carve = [&w](size_t bytes) {
    float *p = reinterpret_cast<float *>(w);
    w += align256(bytes);
    return p;
  };
  BwdArgs a{};
  a.q = q; a.k = k; a.v = v; a.qkv_stride = qkv_row_stride; a.qkv_dtype = qkv_dtype;
  a.g = g; a.g_stride = g_row_stride; a.g_dtype = g_dtype;
  a.beta = beta; a.beta_stride = beta_row_stride; a.beta_dtype = beta_dtype;
  a.A_log = A_log; a.dt_bias = dt_bias; a.scale = scale; a.lb = lower_bound; a.flags = flags;
  a.cu = cu_seqlens; a.n_seqs = n_seqs; a.total = total_tokens; a.num_heads = num_heads;
  a.h0 = initial_state; a.dout = d_out; a.do_stride = d_out_row_stride; a.do_dtype = d_out_dtype;
  a.dht = d_final_state;
  a.dq = dq; a.dk = dk; a.dv = dv; a.dg = dg; a.dbeta = dbeta; a.dh0 = d_initial_state;
  a.grad_dtype = (flags & SOPHIA_KDA_BWD_GRAD_BF16) ? SOPHIA_DTYPE_BF16 : SOPHIA_DTYPE_F32;
  a.dA_log = dA_log; a.ddt_bias = ddt_bias;
  a.qh = carve(tok * kD * 4);
  a.kh = carve(tok * kD * 4);
  a.gl = carve(tok * kD * 4);
  a.bt = carve(tok * 4);
  a.gpb = carve(static_cast<size_t>(kGateParts) * num_heads * kD * 4);
  a.gpa = carve(static_cast<size_t>(kGateParts) * num_heads * kD * 4);
  const bool recurrent = (flags & SOPHIA_KDA_BWD_RECURRENT) != 0;
  if (!recurrent && total_tokens > 0) {
    // the chunk form reads rows of q, k, v and d_out four elements at a time
    const auto aligned = [](const void *ptr, int dtype) {
      return reinterpret_cast<uintptr_t>(ptr) % (dtype == SOPHIA_DTYPE_BF16 ? 8 : 16) == 0;
    };
    SOPHIA_REQUIRE(qkv_row_stride % 4 == 0 && g_row_stride % 4 == 0 && d_out_row_stride % 4 == 0,
                   "kda_chunk_bwd: q/k/v/g/d_out row strides must be multiples of 4 elements");
    SOPHIA_REQUIRE(aligned(q, qkv_dtype) && aligned(k, qkv_dtype) && aligned(v, qkv_dtype) &&
                       aligned(g, g_dtype) && aligned(d_out, d_out_dtype),
                   "kda_chunk_bwd: q/k/v/g/d_out must be aligned to 4 elements");
  }
  void *scratch = nullptr;
  if (recurrent) {
    a.ckpt = carve(max_pieces(total_tokens, n_seqs) * num_heads * kD * kD * 4);
    a.dqh = carve(kSlices * tok * kD * 4);
    a.dkh = carve(kSlices * tok * kD * 4);
    a.dal = carve(kSlices * tok * kD * 4);
    a.dbp = carve(kSlices * tok * 4);
    a.pv = carve(tok * kD * 4);
  } else {
    scratch = carve(chunk_bwd_scratch_bytes(total_tokens, n_seqs, num_heads));
  }
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (recurrent && total_tokens > 0) {
    hipLaunchKernelGGL(kda_bwd_prep_kernel, dim3(static_cast<unsigned>(total_tokens), num_heads), dim3(kD), 0, st,
                       a);
    if (const int rc = check_launch("kda_bwd_prep")) return rc;
  }
  if (recurrent) {
    if (const int rc = ensure_chain_lds()) return rc;
    hipLaunchKernelGGL(kda_bwd_chain_kernel, dim3(static_cast<unsigned>(blocks)), dim3(kChainThreads), kChainLds, st,
                       a);
    if (const int rc = check_launch("kda_bwd_chain")) return rc;
  } else {
    // The chunk form (records, forward states, reverse chunk scan, per-chunk
    // gradients on MFMA, the norms', gate's and sigmoid's backward included):
    // dq, dk, dv, dg, dbeta of every token and dh0.
    ChunkBwdIO io{q, k, v, qkv_row_stride, qkv_dtype, g, g_row_stride, g_dtype, beta, beta_row_stride,
                  beta_dtype, A_log, dt_bias, scale, lower_bound, flags, cu_seqlens, n_seqs, total_tokens,
                  num_heads, initial_state, d_out, d_out_row_stride, d_out_dtype, d_final_state,
                  dq, dk, dg, dbeta, dv, d_initial_state, a.grad_dtype};
    if (const int rc = chunk_bwd_run(io, scratch, st)) return rc;
  }
  if (recurrent && total_tokens > 0) {
    hipLaunchKernelGGL(kda_bwd_post_kernel, dim3(static_cast<unsigned>(total_tokens), num_heads), dim3(kD), 0, st,
                       a);
    if (const int rc = check_launch("kda_bwd_post")) return rc;
  }
  if (recurrent && total_tokens > 0) {
    hipLaunchKernelGGL(kda_bwd_zero_outside_kernel, dim3(kZeroBlocks), dim3(256), 0, st, a);
    if (const int rc = check_launch("kda_bwd_zero_outside")) return rc;
  }
  if (gate && (dA_log || ddt_bias)) {
    hipLaunchKernelGGL(kda_bwd_gate_partial_kernel, dim3(num_heads, kGateParts), dim3(kD), 0, st, a);
    if (const int rc = check_launch("kda_bwd_gate_partial")) return rc;
    hipLaunchKernelGGL(kda_bwd_gate_final_kernel, dim3(num_heads), dim3(kD), 0, st, a);
    if (const int rc = check_launch("kda_bwd_gate_final")) return rc;
  }
  return SOPHIA_OK;
}
