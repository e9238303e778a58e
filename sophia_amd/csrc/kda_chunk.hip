// Chunkwise (C = 64) gated delta-rule prefill over a packed ragged batch, gfx950.
//
// Replaces fla.ops.kda.chunk_kda as called by SophiaKDA._run_kda
// (ml/runtime/model/attention.py:349-365) and its varlen form in FlashKDA
// (ml/training/pretrain/engine/sm120_concurrent_ffn.py:209-268): q/k l2norm,
// in-kernel gate g = lb*sigmoid(exp(A_log)*(z+dt_bias)), beta sigmoid,
// safe gate (g >= -5), chunk 64, state reset at every cu_seqlens boundary.
//
// Per chunk of 64 tokens and head, with G[r] the inclusive within-chunk
// cumulative log-decay, S0 the state entering the chunk:
//   T   = (I + A_kk)^-1,  A_kk[r,j] = beta_r sum_c k_rc k_jc e^{G_rc - G_jc} (j < r)
//   W   = T (beta K e^G),  Ut = T (beta V)
//   U   = Ut - W S0
//   O   = (Q e^G) S0 + A_qk U,  A_qk[r,j] = sum_c q_rc k_jc e^{G_rc - G_jc} (j <= r)
//   S1  = Diag(e^{G_C}) S0 + (K e^{G_C - G})^T U
// Exponents are factorised per 16-token sub-block (reference point at the
// end of the previous sub-block) so that every factor is <= 1, or <= e^80 on
// the diagonal sub-blocks: finite in fp32 and bf16 for g >= -5.
//
// Two kernels:
//  * kda_chunk_intra_kernel (grid: chunk x head, 256 threads): everything that
//    does not depend on S0.  Writes, per (chunk, head), the MFMA operand
//    fragments -W, Q e^G, (K e^{G_C-G})^T, A_qk (bf16, in the exact per-lane
//    order of v_mfma_f32_16x16x32_bf16 A operands), Ut (bf16, C-tile order)
//    and e^{G_C} (fp32) to the workspace.
//  * kda_chunk_scan_kernel (one wavefront per sequence x head x 32 value
//    columns): walks the chunks of its sequence with the fp32 state held in
//    MFMA accumulator tiles.  The C tile of one product is reused as the B
//    operand of the next (16x16x32 operands pair two C tiles; the A operands
//    carry the matching k permutation), so S and U never leave registers.
#include "common.hpp"

namespace sophia {
namespace {

constexpr int kD = 128;   // key / value head dim
constexpr int kC = 64;    // chunk length
constexpr int kThreads = 256;

// ---- workspace record, per (chunk, head) ----------------------------------
constexpr size_t kFrag = 64 * 16;                  // one A fragment: 64 lanes x 8 bf16
constexpr size_t kOffW = 0;                        // -W      [mb 4][ks 4]
constexpr size_t kOffQ = kOffW + 16 * kFrag;       // Q e^G   [mb 4][ks 4]
constexpr size_t kOffKt = kOffQ + 16 * kFrag;      // Kbar^T  [mb 8][ks 2]
constexpr size_t kOffA = kOffKt + 16 * kFrag;      // A_qk    [mb 4][ks 2]
constexpr size_t kOffU = kOffA + 8 * kFrag;        // Ut      [mb 4][nt 8][lane 64][4 bf16]
constexpr size_t kOffG = kOffU + 32 * 64 * 8;      // e^{G_C} [128] fp32
constexpr size_t kRecBytes = kOffG + kD * 4;       // 74240

inline int64_t max_chunks(int64_t total, int n) { return total / kC + n; }
inline size_t header_bytes(int64_t total, int n) {
  size_t b = sizeof(int32_t) * (static_cast<size_t>(n) + 1 + static_cast<size_t>(max_chunks(total, n)));
  return (b + 255) & ~static_cast<size_t>(255);
}

__device__ __forceinline__ f4 mfma32(const bf8 &a, const bf8 &b, const f4 &c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ bf8 pack8(const float *x) {
  bf8 r;
#pragma unroll
  for (int i = 0; i < 8; ++i) r[i] = static_cast<__bf16>(x[i]);
  return r;
}

__device__ __forceinline__ bf8 bits_to_bf8(u4 w) { return __builtin_bit_cast(bf8, w); }
__device__ __forceinline__ u4 bf8_to_bits(bf8 v) { return __builtin_bit_cast(u4, v); }

// Inclusive prefix sum over the 16 lanes of a DPP row.
__device__ __forceinline__ float row_scan16(float x) {
  int v = __float_as_int(x);
  x += __int_as_float(__builtin_amdgcn_update_dpp(0, v, 0x111, 0xf, 0xf, false));
  v = __float_as_int(x);
  x += __int_as_float(__builtin_amdgcn_update_dpp(0, v, 0x112, 0xf, 0xf, false));
  v = __float_as_int(x);
  x += __int_as_float(__builtin_amdgcn_update_dpp(0, v, 0x114, 0xf, 0xf, false));
  v = __float_as_int(x);
  x += __int_as_float(__builtin_amdgcn_update_dpp(0, v, 0x118, 0xf, 0xf, false));
  return x;
}

// Channel held in slot (ks, e) of a lane with lane-group gq: the k order of a
// 16x16x32 operand built from two 16-row C tiles.
__device__ __forceinline__ int perm_k(int ks, int gq, int e) {
  return 32 * ks + 16 * (e >> 2) + 4 * gq + (e & 3);
}

// ---- chunk table -----------------------------------------------------------
// chunk_start[s] = first global chunk of sequence s, chunk_start[n] = total;
// chunk_seq[c] = sequence of global chunk c.
__global__ __launch_bounds__(256) void kda_chunk_prep_kernel(const int32_t *__restrict__ cu, int n,
                                                             int64_t total, int64_t max_ch,
                                                             int32_t *__restrict__ chunk_start,
                                                             int32_t *__restrict__ chunk_seq) {
  __shared__ int32_t part[256];
  const int t = threadIdx.x;
  const int per = (n + 255) / 256;
  const int s0 = min(n, t * per), s1 = min(n, s0 + per);
  auto nchunks = [&](int s) -> int32_t {
    int64_t a = min<int64_t>(max<int64_t>(cu[s], 0), total);
    int64_t b = min<int64_t>(max<int64_t>(cu[s + 1], a), total);
    return static_cast<int32_t>((b - a + kC - 1) / kC);
  };
  int32_t sum = 0;
  for (int s = s0; s < s1; ++s) sum += nchunks(s);
  part[t] = sum;
  __syncthreads();
  for (int off = 1; off < 256; off <<= 1) {
    int32_t v = t >= off ? part[t - off] : 0;
    __syncthreads();
    part[t] += v;
    __syncthreads();
  }
  int32_t base = part[t] - sum;
  for (int s = s0; s < s1; ++s) {
    chunk_start[s] = base;
    const int32_t nc = nchunks(s);
    for (int32_t c = 0; c < nc; ++c)
      if (base + c < max_ch) chunk_seq[base + c] = s;
    base += nc;
  }
  if (t == 255) chunk_start[n] = part[255];
}

// ---- intra-chunk kernel ----------------------------------------------------
// LDS layout (bytes).  sKtT / sVT hold beta K e^G and beta V transposed
// ([channel][row]) with the 16-byte row segments XOR-swizzled by channel.
constexpr int kLdT = 68;    // fp32 row stride of T
constexpr int kLdKD = 136;  // bf16 row stride of K-side rows / -W
constexpr int kLdQK = 72;   // bf16 row stride of A_qk
constexpr size_t kSmTot = 0;                               // float [128][4]: e^{sub-block totals}
constexpr size_t kSmKD = kSmTot + 128 * 4 * 4;             // bf16 [64][136]  (later: -W, solve scratch)
constexpr size_t kSmT = kSmKD + 64 * kLdKD * 2;            // float [64][68]
constexpr size_t kSmQK = kSmT + 64 * kLdT * 4;             // bf16 [64][72]
constexpr size_t kSmKt = kSmQK + 64 * kLdQK * 2;           // bf16 [128][64] swizzled (later: Kbar^T)
constexpr size_t kSmV = kSmKt + 128 * 64 * 2;              // bf16 [128][64] swizzled
constexpr size_t kSmIntra = kSmV + 128 * 64 * 2;           // 78848

__device__ __forceinline__ int swz(int ch, int row) {
  return ch * 64 + ((((row >> 3) ^ (ch & 7))) << 3) + (row & 7);
}

struct IntraArgs {
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
  int64_t max_ch;
  const int32_t *chunk_start, *chunk_seq;
  uint8_t *records;
};

template <int QKV_DT, int G_DT>
__global__ __launch_bounds__(kThreads, 2) void kda_chunk_intra_kernel(IntraArgs p) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  float *s_E = reinterpret_cast<float *>(smem + kSmTot);
  uint16_t *sKD = reinterpret_cast<uint16_t *>(smem + kSmKD);
  float *sT = reinterpret_cast<float *>(smem + kSmT);
  uint16_t *sQK = reinterpret_cast<uint16_t *>(smem + kSmQK);
  uint16_t *sKt = reinterpret_cast<uint16_t *>(smem + kSmKt);
  uint16_t *sV = reinterpret_cast<uint16_t *>(smem + kSmV);
  float *sR = reinterpret_cast<float *>(smem + kSmKD);      // solve scratch [16][48]
  uint16_t *sW = sKD;                                        // -W rows, after the solve

  const int c = blockIdx.x;
  const int h = blockIdx.y;
  const int nch = min<int64_t>(p.chunk_start[p.n_seqs], p.max_ch);
  if (c >= nch) return;
  const int s = p.chunk_seq[c];
  const int64_t seq_a = min<int64_t>(max<int64_t>(p.cu[s], 0), p.total);
  const int64_t seq_b = min<int64_t>(max<int64_t>(p.cu[s + 1], seq_a), p.total);
  const int64_t t0 = seq_a + static_cast<int64_t>(c - p.chunk_start[s]) * kC;
  const int len = static_cast<int>(min<int64_t>(kC, seq_b - t0));

  const int tid = threadIdx.x;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave = 16-row sub-block (uniform)
  const int l = tid & 63;
  const int lr = l & 15;         // row within the sub-block
  const int gq = l >> 4;         // lane group
  const int row = 16 * w + lr;   // chunk row of this lane
  const bool valid = row < len;
  const int64_t tok = t0 + row;

  // ---- 1. load q, k, g (32 channels per lane, 16x16x32 operand order), beta;
  //         beta V goes straight to LDS (transposed), it needs no decay.
  float qv[32], kv[32], gv[32];
  float bt = 0.f;
  if (valid) {
    bt = load_elem(p.beta, tok * p.beta_stride + h, p.beta_dtype);
    if (p.flags & SOPHIA_KDA_BETA_SIGMOID) bt = sigmoid_f(bt);
  }
  {
    const int64_t qrow = tok * p.qkv_stride + static_cast<int64_t>(h) * kD;
    const int64_t grow = tok * p.g_stride + static_cast<int64_t>(h) * kD;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
#pragma unroll
      for (int hf = 0; hf < 2; ++hf) {
        const int ch = 32 * ks + 16 * hf + 4 * gq;
        f4 a = {0.f, 0.f, 0.f, 0.f}, b = a, cc = a, d = a;
        if (valid) {
          a = load4(p.q, qrow + ch, QKV_DT);
          b = load4(p.k, qrow + ch, QKV_DT);
          cc = load4(p.v, qrow + ch, QKV_DT);
          d = load4(p.g, grow + ch, G_DT);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int e = 8 * ks + 4 * hf + i;
          qv[e] = a[i];
          kv[e] = b[i];
          gv[e] = d[i];
          sV[swz(ch + i, row)] = f32_to_bf16_bits(bt * cc[i]);
        }
      }
  }

  // ---- 2. l2 norms (row spread over the 4 lane groups), gate
  {
    float sq = 0.f, sk = 0.f;
#pragma unroll
    for (int e = 0; e < 32; ++e) {
      sq = fmaf(qv[e], qv[e], sq);
      sk = fmaf(kv[e], kv[e], sk);
    }
    sq += __shfl_xor(sq, 16, 64);
    sq += __shfl_xor(sq, 32, 64);
    sk += __shfl_xor(sk, 16, 64);
    sk += __shfl_xor(sk, 32, 64);
    float qs = p.scale, ksc = 1.f;
    if (p.flags & SOPHIA_KDA_QK_L2NORM) {
      qs = p.scale / fmaxf(sqrtf(sq), 1e-12f);
      ksc = 1.f / fmaxf(sqrtf(sk), 1e-12f);
    }
#pragma unroll
    for (int e = 0; e < 32; ++e) {
      qv[e] *= qs;
      kv[e] *= ksc;
    }
    if (p.flags & SOPHIA_KDA_GATE_IN_KERNEL) {
      const float hs = __expf(p.A_log[h]);
#pragma unroll
      for (int e = 0; e < 32; ++e) {
        const int ch = perm_k(e >> 3, gq, e & 7);
        gv[e] = valid ? kda_log_decay(gv[e], hs, p.dt_bias[h * kD + ch], p.lb) : 0.f;
      }
    }
  }

  // ---- 3. within-sub-block cumulative log-decay, sub-block totals
#pragma unroll
  for (int e = 0; e < 32; ++e) gv[e] = row_scan16(gv[e]);
  // s_E[ch][i] = e^{tot_i}: decay over sub-block i (in [e^-80, 1]).
  if (lr == 15) {
#pragma unroll
    for (int e = 0; e < 32; ++e) s_E[perm_k(e >> 3, gq, e & 7) * 4 + w] = __expf(gv[e]);
  }
  __syncthreads();

  // ---- 4. scaled operands; diagonal 16x16 blocks of A_qk / A_kk
  // Per channel, with Gloc the within-sub-block cumulative log-decay and
  // E_i = e^{tot_i}: a = e^{Gloc} (<= 1), b = e^{-Gloc} (<= e^80),
  // d = b E_w (<= 1), eref = e^{ref_w} = prod_{i<w} E_i,
  // etail = e^{G_C - ref_{w+1}} = prod_{i>w} E_i.
  bf8 QSf[4], KSf[4];           // query side, reused for the key block w-1
  u4 kbar_bits[4];              // K e^{G_C - G}, bf16, operand order
  f4 aqk_d = {0.f, 0.f, 0.f, 0.f}, akk_d = aqk_d;
  uint8_t *rec = p.records + (static_cast<size_t>(c) * p.num_heads + h) * kRecBytes;
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
    float qa[8], ka[8], kb[8], kd[8], kbar[8], qe[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int e = 8 * ks + i;
      const int ch = perm_k(ks, gq, i);
      const f4 E = *reinterpret_cast<const f4 *>(&s_E[ch * 4]);
      const float a = __expf(gv[e]);
      const float b = __expf(-gv[e]);
      const float eref = (w > 0 ? E[0] : 1.f) * (w > 1 ? E[1] : 1.f) * (w > 2 ? E[2] : 1.f);
      const float etl = (w < 1 ? E[1] : 1.f) * (w < 2 ? E[2] : 1.f) * (w < 3 ? E[3] : 1.f);
      const float ew = w == 0 ? E[0] : (w == 1 ? E[1] : (w == 2 ? E[2] : E[3]));
      qa[i] = qv[e] * a;
      ka[i] = kv[e] * a;
      kb[i] = kv[e] * b;
      kd[i] = kb[i] * ew;
      kbar[i] = kd[i] * etl;
      qe[i] = qa[i] * eref;                                      // Q e^G
      sKt[swz(ch, row)] = f32_to_bf16_bits(bt * ka[i] * eref);   // beta K e^G
    }
    QSf[ks] = pack8(qa);
    KSf[ks] = pack8(ka);
    const bf8 kbf = pack8(kb);
    aqk_d = mfma32(QSf[ks], kbf, aqk_d);
    akk_d = mfma32(KSf[ks], kbf, akk_d);
    kbar_bits[ks] = bf8_to_bits(pack8(kbar));
    // Q e^G goes straight to the workspace in A-operand order (mb = w).
    *reinterpret_cast<u4 *>(rec + kOffQ + ((w * 4 + ks) * 64 + l) * 16) = bf8_to_bits(pack8(qe));
    // K-side rows for the off-diagonal blocks, row-major bf16.
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
      u2 wv;
      wv.x = pack_bf16x2(kd[4 * hf], kd[4 * hf + 1]);
      wv.y = pack_bf16x2(kd[4 * hf + 2], kd[4 * hf + 3]);
      *reinterpret_cast<u2 *>(&sKD[row * kLdKD + 32 * ks + 16 * hf + 4 * gq]) = wv;
    }
    __builtin_amdgcn_sched_barrier(0);  // keep the next K-step's LDS reads from being hoisted
  }
  __syncthreads();

  // ---- 5. off-diagonal blocks of A_qk / A_kk for query sub-block w
  // Key block ib < w: A_*[r, j] = sum_c (q,k)_r e^{Gloc_r} f_c KD_j with
  // f = e^{ref_w - ref_{ib+1}} = prod_{ib<i<w} E_i (<= 1, 1 for ib = w-1).
  {
    float brow[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) brow[e] = __shfl(bt, 4 * gq + e, 64);
#pragma unroll 1
    for (int ib = 0; ib < 4; ++ib) {
      f4 aqk = aqk_d, akk = akk_d;
      if (ib != w) aqk = akk = f4{0.f, 0.f, 0.f, 0.f};
      if (ib == w - 1) {
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
          const uint16_t *src = &sKD[(16 * ib + lr) * kLdKD + 32 * ks + 4 * gq];
          const u2 lo = *reinterpret_cast<const u2 *>(src);
          const u2 hi = *reinterpret_cast<const u2 *>(src + 16);
          const bf8 bk = bits_to_bf8(u4{lo.x, lo.y, hi.x, hi.y});
          aqk = mfma32(QSf[ks], bk, aqk);
          akk = mfma32(KSf[ks], bk, akk);
        }
      } else if (ib < w - 1) {
#pragma unroll 1
        for (int ks = 0; ks < 4; ++ks) {
          const uint16_t *src = &sKD[(16 * ib + lr) * kLdKD + 32 * ks + 4 * gq];
          const u2 lo = *reinterpret_cast<const u2 *>(src);
          const u2 hi = *reinterpret_cast<const u2 *>(src + 16);
          const bf8 bk = bits_to_bf8(u4{lo.x, lo.y, hi.x, hi.y});
          const bf8 aq0 = QSf[ks], ak0 = KSf[ks];
          float tq[8], tk[8];
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            const f4 E = *reinterpret_cast<const f4 *>(&s_E[perm_k(ks, gq, i) * 4]);
            const float e1 = w == 2 ? E[1] : E[2];             // E_{w-1}, w in {2, 3}
            const float f = (ib == w - 2) ? e1 : E[1] * E[2];     // w = 3, ib = 0
            tq[i] = static_cast<float>(aq0[i]) * f;
            tk[i] = static_cast<float>(ak0[i]) * f;
          }
          aqk = mfma32(pack8(tq), bk, aqk);
          akk = mfma32(pack8(tk), bk, akk);
        }
      }
      // C tile: rows 16w + 4gq + e, column 16ib + lr.
      const int col = 16 * ib + lr;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int r = 16 * w + 4 * gq + e;
        sQK[r * kLdQK + col] = f32_to_bf16_bits(col <= r ? aqk[e] : 0.f);
        sT[r * kLdT + col] = col < r ? akk[e] * brow[e] : 0.f;
      }
    }
  }
  __syncthreads();

  // ---- 6. T = (I + A_kk)^-1 (fp32), 16x16 diagonal inverses then block rows
  {
    float x[16];
    if (l < 16) {
      const int n = l;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        float acc = (r == n) ? 1.f : 0.f;
#pragma unroll
        for (int j = 0; j < r; ++j) acc = fmaf(-sT[(16 * w + r) * kLdT + 16 * w + j], x[j], acc);
        x[r] = acc;
      }
    }
    __syncthreads();
    if (l < 16) {
#pragma unroll
      for (int r = 0; r < 16; ++r) sT[(16 * w + r) * kLdT + 16 * w + l] = x[r];
    }
    __syncthreads();
    for (int ib = 1; ib < 4; ++ib) {
      // R = sum_{kb=jb}^{ib-1} L[ib][kb] X[kb][jb]  for columns 0 .. 16 ib - 1
      for (int idx = tid; idx < 16 * 16 * ib; idx += kThreads) {
        const int ri = idx / (16 * ib), cj = idx % (16 * ib);
        const int m0 = 16 * (cj >> 4);
        float acc = 0.f;
        for (int m = m0; m < 16 * ib; ++m) acc = fmaf(sT[(16 * ib + ri) * kLdT + m], sT[m * kLdT + cj], acc);
        sR[ri * 48 + cj] = acc;
      }
      __syncthreads();
      for (int idx = tid; idx < 16 * 16 * ib; idx += kThreads) {
        const int ri = idx / (16 * ib), cj = idx % (16 * ib);
        float acc = 0.f;
        for (int m = 0; m <= ri; ++m) acc = fmaf(sT[(16 * ib + ri) * kLdT + 16 * ib + m], sR[m * 48 + cj], acc);
        sT[(16 * ib + ri) * kLdT + cj] = -acc;
      }
      __syncthreads();
    }
  }

  // ---- 7. W = T (beta K e^G), Ut = T (beta V) for rows 16w .. 16w+15
  {
    f4 accW[8], accU[8];
#pragma unroll
    for (int nt = 0; nt < 8; ++nt) accW[nt] = accU[nt] = f4{0.f, 0.f, 0.f, 0.f};
    const int nks = (w < 2) ? 1 : 2;
    for (int ks = 0; ks < nks; ++ks) {
      const float *tr = &sT[(16 * w + lr) * kLdT + 32 * ks + 8 * gq];
      float ta[8];
      const f4 t0v = *reinterpret_cast<const f4 *>(tr);
      const f4 t1v = *reinterpret_cast<const f4 *>(tr + 4);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        ta[i] = t0v[i];
        ta[4 + i] = t1v[i];
      }
      const bf8 af = pack8(ta);
#pragma unroll
      for (int nt = 0; nt < 8; ++nt) {
        const int ch = 16 * nt + lr;
        const bf8 bk = bits_to_bf8(*reinterpret_cast<const u4 *>(&sKt[swz(ch, 32 * ks + 8 * gq)]));
        const bf8 bv = bits_to_bf8(*reinterpret_cast<const u4 *>(&sV[swz(ch, 32 * ks + 8 * gq)]));
        accW[nt] = mfma32(af, bk, accW[nt]);
        accU[nt] = mfma32(af, bv, accU[nt]);
      }
    }
    // Ut in C-tile order; -W row-major into LDS.
#pragma unroll
    for (int nt = 0; nt < 8; ++nt) {
      u2 uw;
      uw.x = pack_bf16x2(accU[nt][0], accU[nt][1]);
      uw.y = pack_bf16x2(accU[nt][2], accU[nt][3]);
      *reinterpret_cast<u2 *>(rec + kOffU + ((w * 8 + nt) * 64 + l) * 8) = uw;
#pragma unroll
      for (int e = 0; e < 4; ++e)
        sW[(16 * w + 4 * gq + e) * kLdKD + 16 * nt + lr] = f32_to_bf16_bits(-accW[nt][e]);
    }
  }
  __syncthreads();

  // ---- 8. Kbar^T (transposed into the sKt region) and e^{G_C}
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
    const u4 kw = kbar_bits[ks];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t word = kw[i >> 1];
      sKt[swz(perm_k(ks, gq, i), row)] = static_cast<uint16_t>((i & 1) ? (word >> 16) : (word & 0xffffu));
    }
  }
  if (tid < kD) {
    const f4 E = *reinterpret_cast<const f4 *>(&s_E[tid * 4]);
    reinterpret_cast<float *>(rec + kOffG)[tid] = E[0] * E[1] * E[2] * E[3];
  }
  __syncthreads();

  // ---- 9. A-operand fragments from LDS to the workspace
  // -W: m = chunk rows 16w + lr, k = channels perm_k(ks, gq, .)
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
    const uint16_t *src = &sW[(16 * w + lr) * kLdKD + 32 * ks + 4 * gq];
    const u2 lo = *reinterpret_cast<const u2 *>(src);
    const u2 hi = *reinterpret_cast<const u2 *>(src + 16);
    u4 o = {lo.x, lo.y, hi.x, hi.y};
    *reinterpret_cast<u4 *>(rec + kOffW + ((w * 4 + ks) * 64 + l) * 16) = o;
  }
  // Kbar^T: m = channels 16mb + lr (mb = 2w, 2w+1), k = chunk rows perm_k(ks, gq, .)
#pragma unroll
  for (int mi = 0; mi < 2; ++mi) {
    const int mb = 2 * w + mi;
    const int ch = 16 * mb + lr;
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const int r0 = 32 * ks + 4 * gq;
      const u2 lo = *reinterpret_cast<const u2 *>(&sKt[swz(ch, r0)]);
      const u2 hi = *reinterpret_cast<const u2 *>(&sKt[swz(ch, r0 + 16)]);
      u4 o = {lo.x, lo.y, hi.x, hi.y};
      *reinterpret_cast<u4 *>(rec + kOffKt + ((mb * 2 + ks) * 64 + l) * 16) = o;
    }
  }
  // A_qk: m = chunk rows 16w + lr, k = chunk rows perm_k(ks, gq, .)
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) {
    const uint16_t *src = &sQK[(16 * w + lr) * kLdQK + 32 * ks + 4 * gq];
    const u2 lo = *reinterpret_cast<const u2 *>(src);
    const u2 hi = *reinterpret_cast<const u2 *>(src + 16);
    u4 o = {lo.x, lo.y, hi.x, hi.y};
    *reinterpret_cast<u4 *>(rec + kOffA + ((w * 2 + ks) * 64 + l) * 16) = o;
  }
}

// ---- scan kernel -------------------------------------------------------------
struct ScanArgs {
  const int32_t *cu;
  int n_seqs;
  int64_t total;
  int num_heads;
  int64_t max_ch;
  const int32_t *chunk_start;
  const uint8_t *records;
  const float *h0;
  float *ht;
  int n_slots;
  const int32_t *slots;
  void *o;
  int64_t o_stride;
  int o_dtype;
};

// One wavefront per (sequence, head, NV value columns); 4 wavefronts per block.
template <int NV, int O_DT>
__global__ __launch_bounds__(kThreads) void kda_chunk_scan_kernel(ScanArgs p) {
  constexpr int NT = NV / 16;                 // 16-column tiles per wave
  constexpr int WAVES_PER_HEAD = kD / NV;
  const int l = threadIdx.x & 63;
  const int lr = l & 15, gq = l >> 4;
  const int gw = blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6);
  const int vt = gw % WAVES_PER_HEAD;
  const int sh = gw / WAVES_PER_HEAD;
  const int h = sh % p.num_heads;
  const int s = sh / p.num_heads;
  if (s >= p.n_seqs) return;
  const int v0 = vt * NV;
  const int64_t seq_a = min<int64_t>(max<int64_t>(p.cu[s], 0), p.total);
  const int64_t seq_b = min<int64_t>(max<int64_t>(p.cu[s + 1], seq_a), p.total);
  const int nchunks = static_cast<int>((seq_b - seq_a + kC - 1) / kC);
  const int cbase = p.chunk_start[s];
  const int slot = p.slots ? p.slots[s] : s;
  const bool has_slot = slot >= 0 && slot < p.n_slots;  // else: zero start, nothing written
  const int64_t state_off = (static_cast<int64_t>(has_slot ? slot : 0) * p.num_heads + h) * kD * kD;

  // S tiles: [mb 8][nt NT], lane holds rows 16mb + 4gq + e, column v0 + 16nt + lr.
  f4 S[8][NT];
#pragma unroll
  for (int mb = 0; mb < 8; ++mb)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      f4 v = {0.f, 0.f, 0.f, 0.f};
      if (p.h0 && has_slot) {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          v[e] = p.h0[state_off + static_cast<int64_t>(16 * mb + 4 * gq + e) * kD + v0 + 16 * nt + lr];
      }
      S[mb][nt] = v;
    }

  for (int cc = 0; cc < nchunks; ++cc) {
    const int64_t gc = cbase + cc;
    if (gc >= p.max_ch) break;
    const uint8_t *rec = p.records + (static_cast<size_t>(gc) * p.num_heads + h) * kRecBytes;

    // S as bf16 B operands: K-step ks pairs tiles 2ks and 2ks+1.
    bf8 Sb[4][NT];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        float t[8];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          t[e] = S[2 * ks][nt][e];
          t[4 + e] = S[2 * ks + 1][nt][e];
        }
        Sb[ks][nt] = pack8(t);
      }

    // U = Ut - W S
    f4 U[4][NT];
#pragma unroll
    for (int mb = 0; mb < 4; ++mb) {
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        const u2 uw = *reinterpret_cast<const u2 *>(rec + kOffU + ((mb * 8 + v0 / 16 + nt) * 64 + l) * 8);
        U[mb][nt] = f4{__uint_as_float(uw.x << 16), __uint_as_float(uw.x & 0xffff0000u),
                       __uint_as_float(uw.y << 16), __uint_as_float(uw.y & 0xffff0000u)};
      }
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const bf8 a = bits_to_bf8(*reinterpret_cast<const u4 *>(rec + kOffW + ((mb * 4 + ks) * 64 + l) * 16));
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) U[mb][nt] = mfma32(a, Sb[ks][nt], U[mb][nt]);
      }
    }
    bf8 Ub[2][NT];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        float t[8];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          t[e] = U[2 * ks][nt][e];
          t[4 + e] = U[2 * ks + 1][nt][e];
        }
        Ub[ks][nt] = pack8(t);
      }

    // O = (Q e^G) S + A_qk U, stored for the valid rows of the chunk.
    const int64_t tok0 = seq_a + static_cast<int64_t>(cc) * kC;
    const int rows_valid = static_cast<int>(min<int64_t>(kC, seq_b - tok0));
#pragma unroll
    for (int mb = 0; mb < 4; ++mb) {
      f4 O[NT];
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) O[nt] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const bf8 a = bits_to_bf8(*reinterpret_cast<const u4 *>(rec + kOffQ + ((mb * 4 + ks) * 64 + l) * 16));
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) O[nt] = mfma32(a, Sb[ks][nt], O[nt]);
      }
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        if (ks == 1 && mb < 2) continue;  // A_qk is lower triangular
        const bf8 a = bits_to_bf8(*reinterpret_cast<const u4 *>(rec + kOffA + ((mb * 2 + ks) * 64 + l) * 16));
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) O[nt] = mfma32(a, Ub[ks][nt], O[nt]);
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int r = 16 * mb + 4 * gq + e;
        if (r < rows_valid) {
          const int64_t base = (tok0 + r) * p.o_stride + static_cast<int64_t>(h) * kD + v0 + lr;
#pragma unroll
          for (int nt = 0; nt < NT; ++nt) store_elem(p.o, base + 16 * nt, O_DT, O[nt][e]);
        }
      }
    }

    // S = Diag(e^{G_C}) S + Kbar^T U
    const float *gam = reinterpret_cast<const float *>(rec + kOffG);
#pragma unroll
    for (int mb = 0; mb < 8; ++mb) {
      const f4 gm = *reinterpret_cast<const f4 *>(&gam[16 * mb + 4 * gq]);
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) S[mb][nt] *= gm;
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const bf8 a = bits_to_bf8(*reinterpret_cast<const u4 *>(rec + kOffKt + ((mb * 2 + ks) * 64 + l) * 16));
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) S[mb][nt] = mfma32(a, Ub[ks][nt], S[mb][nt]);
      }
    }
  }

  if (p.ht && has_slot) {
#pragma unroll
    for (int mb = 0; mb < 8; ++mb)
#pragma unroll
      for (int nt = 0; nt < NT; ++nt)
#pragma unroll
        for (int e = 0; e < 4; ++e)
          p.ht[state_off + static_cast<int64_t>(16 * mb + 4 * gq + e) * kD + v0 + 16 * nt + lr] = S[mb][nt][e];
  }
}

constexpr int kScanNV = 32;

template <int QKV_DT, int G_DT>
int launch_intra(dim3 grid, hipStream_t st, const IntraArgs &ia) {
  static bool attr_set = false;
  if (!attr_set) {
    hipError_t e = hipFuncSetAttribute(
        reinterpret_cast<const void *>(&kda_chunk_intra_kernel<QKV_DT, G_DT>),
        hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(kSmIntra));
    if (e != hipSuccess)
      return set_error(SOPHIA_ERR_HIP, "kda_chunk_fwd: cannot set LDS size: %s", hipGetErrorString(e));
    attr_set = true;
  }
  hipLaunchKernelGGL((kda_chunk_intra_kernel<QKV_DT, G_DT>), grid, dim3(kThreads), kSmIntra, st, ia);
  return check_launch("kda_chunk_intra");
}

}  // namespace
}  // namespace sophia

using namespace sophia;

extern "C" size_t sophia_kda_chunk_workspace_size(int64_t total_tokens, int n_seqs, int num_heads,
                                                  int head_dim) {
  if (total_tokens < 0 || n_seqs <= 0 || num_heads <= 0 || head_dim != kD) return 0;
  return header_bytes(total_tokens, n_seqs) +
         static_cast<size_t>(max_chunks(total_tokens, n_seqs)) * num_heads * kRecBytes;
}

extern "C" int sophia_kda_chunk_fwd(const void *q, const void *k, const void *v,
                                    int64_t qkv_row_stride, int qkv_dtype, const void *g,
                                    int64_t g_row_stride, int g_dtype, const void *beta,
                                    int64_t beta_row_stride, int beta_dtype, const float *A_log,
                                    const float *dt_bias, float scale, float lower_bound,
                                    unsigned flags, const int32_t *cu_seqlens, int n_seqs,
                                    int64_t total_tokens, int num_heads, int head_dim,
                                    const float *initial_state, float *final_state,
                                    int n_state_slots, const int32_t *state_slots, void *o,
                                    int64_t o_row_stride,
                                    void *workspace, size_t workspace_bytes, void *stream) {
  SOPHIA_REQUIRE(head_dim == kD, "kda_chunk_fwd: head_dim must be 128 (got %d)", head_dim);
  SOPHIA_REQUIRE(n_seqs > 0 && num_heads > 0 && num_heads <= 65535 && total_tokens >= 0,
                 "kda_chunk_fwd: bad n_seqs / num_heads / total_tokens");
  SOPHIA_REQUIRE(qkv_dtype == SOPHIA_DTYPE_F32 || qkv_dtype == SOPHIA_DTYPE_BF16,
                 "kda_chunk_fwd: qkv dtype %d not supported", qkv_dtype);
  SOPHIA_REQUIRE(g_dtype == SOPHIA_DTYPE_F32 || g_dtype == SOPHIA_DTYPE_BF16,
                 "kda_chunk_fwd: g dtype %d not supported", g_dtype);
  SOPHIA_REQUIRE(beta_dtype == SOPHIA_DTYPE_F32 || beta_dtype == SOPHIA_DTYPE_BF16,
                 "kda_chunk_fwd: beta dtype %d not supported", beta_dtype);
  SOPHIA_REQUIRE(cu_seqlens && workspace && (total_tokens == 0 || (q && k && v && g && beta && o)),
                 "kda_chunk_fwd: NULL pointer");
  SOPHIA_REQUIRE(!(flags & SOPHIA_KDA_GATE_IN_KERNEL) || (A_log && dt_bias),
                 "kda_chunk_fwd: gate in kernel needs A_log and dt_bias");
  SOPHIA_REQUIRE(lower_bound >= -5.0f && lower_bound < 0.0f,
                 "kda_chunk_fwd: lower_bound must be in [-5, 0) (safe gate range)");
  SOPHIA_REQUIRE(qkv_row_stride >= (int64_t)num_heads * kD && g_row_stride >= (int64_t)num_heads * kD &&
                     beta_row_stride >= num_heads && o_row_stride >= (int64_t)num_heads * kD,
                 "kda_chunk_fwd: row stride smaller than a row");
  SOPHIA_REQUIRE(qkv_row_stride % 4 == 0 && g_row_stride % 4 == 0,
                 "kda_chunk_fwd: q/k/v/g row strides must be multiples of 4 elements");
  SOPHIA_REQUIRE(((uintptr_t)workspace % 256) == 0, "kda_chunk_fwd: workspace must be 256-byte aligned");
  SOPHIA_REQUIRE(n_state_slots >= 0, "kda_chunk_fwd: n_state_slots must be >= 0");
  const size_t need = sophia_kda_chunk_workspace_size(total_tokens, n_seqs, num_heads, head_dim);
  if (workspace_bytes < need)
    return set_error(SOPHIA_ERR_WORKSPACE, "kda_chunk_fwd: workspace %zu bytes < required %zu",
                     workspace_bytes, need);
  const int64_t max_ch = max_chunks(total_tokens, n_seqs);
  SOPHIA_REQUIRE(max_ch <= 0x7fffffff, "kda_chunk_fwd: too many chunks");
  hipStream_t st = static_cast<hipStream_t>(stream);
  int32_t *chunk_start = static_cast<int32_t *>(workspace);
  int32_t *chunk_seq = chunk_start + n_seqs + 1;
  uint8_t *records = static_cast<uint8_t *>(workspace) + header_bytes(total_tokens, n_seqs);

  hipLaunchKernelGGL(kda_chunk_prep_kernel, dim3(1), dim3(256), 0, st, cu_seqlens, n_seqs,
                     total_tokens, max_ch, chunk_start, chunk_seq);
  int rc = check_launch("kda_chunk_prep");
  if (rc) return rc;

  if (max_ch > 0 && total_tokens > 0) {
    IntraArgs ia{q, k, v, qkv_row_stride, qkv_dtype, g, g_row_stride, g_dtype, beta,
                 beta_row_stride, beta_dtype, A_log, dt_bias, scale, lower_bound, flags,
                 cu_seqlens, n_seqs, total_tokens, num_heads, max_ch, chunk_start, chunk_seq,
                 records};
    const dim3 grid(static_cast<unsigned>(max_ch), num_heads);
    if (qkv_dtype == SOPHIA_DTYPE_BF16 && g_dtype == SOPHIA_DTYPE_F32)
      rc = launch_intra<SOPHIA_DTYPE_BF16, SOPHIA_DTYPE_F32>(grid, st, ia);
    else if (qkv_dtype == SOPHIA_DTYPE_BF16)
      rc = launch_intra<SOPHIA_DTYPE_BF16, SOPHIA_DTYPE_BF16>(grid, st, ia);
    else if (g_dtype == SOPHIA_DTYPE_F32)
      rc = launch_intra<SOPHIA_DTYPE_F32, SOPHIA_DTYPE_F32>(grid, st, ia);
    else
      rc = launch_intra<SOPHIA_DTYPE_F32, SOPHIA_DTYPE_BF16>(grid, st, ia);
    if (rc) return rc;
  }
  ScanArgs sa{cu_seqlens, n_seqs, total_tokens, num_heads, max_ch, chunk_start, records,
              initial_state, final_state, n_state_slots, state_slots, o, o_row_stride, qkv_dtype};
  const int64_t waves = static_cast<int64_t>(n_seqs) * num_heads * (kD / kScanNV);
  const int64_t blocks = (waves + 3) / 4;
  SOPHIA_REQUIRE(blocks <= 0x7fffffff, "kda_chunk_fwd: grid too large");
  if (qkv_dtype == SOPHIA_DTYPE_BF16)
    hipLaunchKernelGGL((kda_chunk_scan_kernel<kScanNV, SOPHIA_DTYPE_BF16>),
                       dim3(static_cast<unsigned>(blocks)), dim3(kThreads), 0, st, sa);
  else
    hipLaunchKernelGGL((kda_chunk_scan_kernel<kScanNV, SOPHIA_DTYPE_F32>),
                       dim3(static_cast<unsigned>(blocks)), dim3(kThreads), 0, st, sa);
  return check_launch("kda_chunk_scan");
}
