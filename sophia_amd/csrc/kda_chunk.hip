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
//  * kda_chunk_intra_kernel (one 256-thread work-group per (chunk, head),
//    heads fastest): everything that does not depend on S0.  Writes, per
//    (chunk, head), the MFMA operand fragments -W, Q e^G, (K e^{G_C-G})^T,
//    A_qk (bf16, in the exact per-lane order of v_mfma_f32_16x16x32_bf16 A
//    operands), Ut (bf16, C-tile order) and e^{G_C} (fp32) to the workspace.
//  * kda_chunk_scan_kernel (one work-group of 8 wavefronts per sequence x
//    head x 128/splits value columns): walks the chunks of its sequence.  Four
//    wavefronts hold the fp32 state in MFMA accumulator tiles and update it;
//    four form U and O.  S and U pass between them through LDS as bf16 MFMA
//    operands (16x16x32 operands pair two C tiles; the A operands carry the
//    matching k permutation).
#include <algorithm>
#include <mutex>

#include "common.hpp"
#include "kda_chunk_bwd.hpp"
#include "kda_plan.hpp"

namespace sophia {
namespace {

constexpr int kD = 128;   // key / value head dim
constexpr int kC = 64;    // chunk length
static_assert(kC == plan::kChunk, "the launch plans count chunks of kC tokens");
using plan::kMaxClasses;
using plan::kOrderMax;
using plan::kSegChunks;
using plan::kSegSeqMax;
using plan::max_segments;
using plan::plan_scan;
using plan::plan_segments;
using plan::ScanPlan;
using plan::SegPlan;
constexpr int kThreads = 256;
constexpr float kLog2e = 1.4426950408889634f;

// ---- workspace record, per (chunk, head) ----------------------------------
constexpr size_t kFrag = 64 * 16;                  // one A fragment: 64 lanes x 8 bf16
constexpr size_t kOffW = 0;                        // -W      [mb 4][ks 4]
constexpr size_t kOffQ = kOffW + 16 * kFrag;       // Q e^G   [mb 4][ks 4]
constexpr size_t kOffKt = kOffQ + 16 * kFrag;      // Kbar^T  [mb 8][ks 2]
constexpr size_t kOffA = kOffKt + 16 * kFrag;      // A_qk    [mb 4][ks 2]
constexpr size_t kOffU = kOffA + 8 * kFrag;        // Ut      [mb 4][nt 8][lane 64][4 bf16]
constexpr size_t kOffG = kOffU + 32 * 64 * 8;      // e^{G_C} [128] fp32
constexpr size_t kRecBytes = kOffG + kD * 4;       // 74240

// ---- backward record, per (chunk, head) (the backward's instantiation of
// the intra kernel writes it beside the forward record) -------------------
//  Kbar   A operand, m = chunk rows 16mb + lr, k = channels perm_k   [mb 4][ks 4]
//  Qg^T   A operand, m = channels 16mb + lr, k = chunk rows perm_k [mb 8][ks 2]
//  -W^T   A operand, m = channels, k = chunk rows perm_k           [mb 8][ks 2]
//  A_qk^T A operand, m = chunk rows j 16mb + lr, k = rows i perm_k [mb 4][ks 2]
//  dO     B operand, k = chunk rows perm_k, n = value cols 16nt+lr [ks 2][nt 8]
constexpr size_t kBOffKbar = 0;
constexpr size_t kBOffQt = kBOffKbar + 16 * kFrag;
constexpr size_t kBOffWt = kBOffQt + 16 * kFrag;
constexpr size_t kBOffAt = kBOffWt + 16 * kFrag;
constexpr size_t kBOffDo = kBOffAt + 8 * kFrag;
constexpr size_t kBwdRecBytes = kBOffDo + 16 * kFrag;   // 73728

inline int64_t max_chunks(int64_t total, int n) { return total / kC + n; }
// Scratch rows for the stores of chunk rows past the end of a sequence
// (64 rows x 128 fp32 columns, contents never read).
constexpr size_t kTrashBytes = kC * kD * 4;


__device__ __forceinline__ f4 mfma32(const bf8 &a, const bf8 &b, const f4 &c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// fp32 16x16x4 MFMA: lane l supplies a[l % 16][k] and b[k][l % 16] for k slot
// l / 16; c holds rows 4 (l / 16) + i, column l % 16.
__device__ __forceinline__ f4 mfma_f32x4(float a, float b, const f4 &c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
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

// ---- chunk numbering -------------------------------------------------------
// Chunks are numbered sequence by sequence, ceil(len / 64) per sequence.  Each
// wavefront finds what it needs by a scan over cu_seqlens (64 sequences per
// step), so no chunk table is built before the kernels; every lane gets the
// same (wavefront-uniform) answer.  Offsets are clamped into [0, total] and
// made monotone, so malformed cu_seqlens never move an access out of bounds.
__device__ __forceinline__ int chunks_of_lane(const int32_t *cu, int n, int64_t total, int s) {
  if (s >= n) return 0;
  const int64_t a = iclamp64(cu[s], 0, total);
  const int64_t b = iclamp64(cu[s + 1], a, total);
  return static_cast<int>((b - a + kC - 1) / kC);
}

__device__ __forceinline__ int wave_incl_scan(int v, int lane) {
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int u = __shfl_up(v, off, 64);
    if (lane >= off) v += u;
  }
  return v;
}

// Sequence s of global chunk c and the number of the sequence's first chunk;
// s = n when c is past the last chunk.
__device__ __forceinline__ void chunk_of(const int32_t *cu, int n, int64_t total, int c, int &s_out,
                                         int &first_out) {
  const int lane = threadIdx.x & 63;
  int done = 0;
  for (int s0 = 0; s0 < n; s0 += 64) {
    const int cnt = chunks_of_lane(cu, n, total, s0 + lane);
    const int incl = wave_incl_scan(cnt, lane);
    const uint64_t hit = __ballot(s0 + lane < n && c < done + incl);
    if (hit) {
      const int l = __builtin_ctzll(hit);
      s_out = s0 + l;
      first_out = done + __shfl(incl - cnt, l, 64);
      return;
    }
    done += __shfl(incl, 63, 64);
  }
  s_out = n;
  first_out = done;
}

// Number of the first chunk of sequence s (the chunks of the sequences before it).
__device__ __forceinline__ int first_chunk(const int32_t *cu, int n, int64_t total, int s) {
  const int lane = threadIdx.x & 63;
  int done = 0;
  for (int s0 = 0; s0 < s; s0 += 64) {
    const int cnt = s0 + lane < s ? chunks_of_lane(cu, n, total, s0 + lane) : 0;
    done += __shfl(wave_incl_scan(cnt, lane), 63, 64);
  }
  return done;
}

// ---- intra-chunk kernel ----------------------------------------------------
// The inputs are read once, with the non-temporal hint, so that they do not
// take the place of the records in the last-level cache (MALL, 256 MB): the
// records are written with ordinary stores and the scan reads them back from
// it where they are still there.  Work-groups take the chunks last first, so
// the first chunks of every sequence, which the scan reads first, are the most
// recently written.  On the 8-sequence benchmark batch (236 MB of records)
// the scan that follows runs 87 -> 71 us against non-temporal record stores in
// chunk order; ordinary input loads instead push it to 95 us.
// LDS regions (bytes).  Lifetimes (steps below) let regions A and B be reused.
//  E: e^{sub-block totals}          float [128][4]           steps 3-8
//  A: key-side rows KD (6 copies)   bf16  [96][136]           steps 4-5
//     -> beta K e^G, transposed     bf16  [128][64] swizzled  steps 7-8
//  B: beta V, transposed            bf16  [128][64] swizzled  steps 1-8
//  C: Kbar, transposed              bf16  [128][64] swizzled  steps 4-4b
//     -> A_kk -> T = (I + A_kk)^-1  float [64][68]            steps 5-8
//  D: A_qk                          bf16  [64][72]            steps 5-10
//  backward instantiation, after step 9: A <- Q e^G transposed, B <- dO
//  transposed (swizzled [128][64] bf16 each), read into the backward record
constexpr int kLdT = 68;    // fp32 row stride of T
constexpr int kLdKD = 136;  // bf16 row stride of key-side rows / -W
constexpr int kLdQK = 72;   // bf16 row stride of A_qk
constexpr size_t kSmE = 0;
constexpr size_t kSmA = kSmE + 128 * 4 * 4;
constexpr size_t kSmB = kSmA + 96 * kLdKD * 2;
constexpr size_t kSmC = kSmB + 64 * kLdKD * 2;
constexpr size_t kSmD = kSmC + 64 * kLdT * 4;
constexpr size_t kSmIntra = kSmD + 64 * kLdQK * 2;           // 73216
// The backward's instantiation transposes Q e^G and dO through regions A and
// B after their last use (step 9), so it needs no more LDS than the forward.
constexpr size_t kSmIntraBwd = kSmIntra;
static_assert(128 * 64 * 2 <= 96 * kLdKD * 2, "region A holds a swizzled [128][64] bf16 tile");
static_assert(128 * 64 * 2 <= 64 * kLdKD * 2, "region B holds a swizzled [128][64] bf16 tile");
static_assert(128 * 64 * 2 <= 64 * kLdT * 4, "region C holds a swizzled [128][64] bf16 tile");
// Step 1 stages whole-line q, k, v rows, 4 KB per wave and tensor, where no
// wave writes before step 3: q in region A, k in region C, v in the rest of A
// (waves 0, 1) and in region D (waves 2, 3).
__device__ __forceinline__ size_t stage_v(int w) { return w < 2 ? kSmA + 16384 + w * 4096 : kSmD + (w - 2) * 4096; }
static_assert(16384 + 2 * 4096 <= 96 * kLdKD * 2 && 2 * 4096 <= 64 * kLdQK * 2 && 4 * 4096 <= 64 * kLdT * 4,
              "step-1 staging fits regions A, C and D");

__device__ __forceinline__ int swz(int ch, int row) {
  return ch * 64 + ((((row >> 3) ^ (ch & 7))) << 3) + (row & 7);
}

// Row block of region A holding key block ib scaled for query block ib+1+v
// (v = 0: KD itself, v = 1: KD E_{ib+1}, v = 2: KD E_{ib+1} E_{ib+2}).
__device__ __forceinline__ int kd_slot(int ib, int v) { return v == 0 ? ib : (v == 1 ? 3 + ib : 5); }

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
  uint8_t *records;
  int qkv_lines;  // bf16 q/k/v with 16-byte aligned rows: load whole lines through LDS
  // Backward instantiations only: the backward record, T = (I + A_kk)^-1 and
  // P = A_kk / beta in one fp32 [64][64] tile per (chunk, head) (T[r][c] at
  // [r][c] for c <= r, P[r][c] at [c][r] for c < r), and the output gradient.
  uint8_t *brec;
  float *tpmat;
  const void *dout;
  int64_t do_stride;
  int do_dtype;
  // Fused ShortConv instantiations only (kda_chunk_conv_intra_kernel): q, k,
  // v above are the rows before the conv; taps [3 H 128][4] fp32 (q | k | v
  // channels, taps[c][3] multiplies the current row); histories
  // [conv_n_slots][3 H 128][3] fp32, sequence s in slot conv_slots[s] (or s),
  // read when conv_read (else, and for a slot out of range, zeros).
  const float *conv_w;
  float *conv_state;
  const int32_t *conv_slots;
  int conv_n_slots;
  int conv_read;
};

__device__ __forceinline__ float fast_sigmoid(float x) {
  return __builtin_amdgcn_rcpf(1.0f + __expf(-x));
}

__device__ __forceinline__ u2 pack4_bf16(f4 v) {
  return u2{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
}

// Four consecutive elements as loaded from memory (bf16 pairs or fp32),
// converted to fp32 only when used, so that loads can be batched.
template <int DT>
struct Raw4;
template <>
struct Raw4<SOPHIA_DTYPE_BF16> {
  u2 w;
  __device__ __forceinline__ void load(const void *base, int64_t idx) {
    w = *reinterpret_cast<const u2 *>(static_cast<const uint16_t *>(base) + idx);
  }
  __device__ __forceinline__ f4 get() const {
    return f4{__uint_as_float(w.x << 16), __uint_as_float(w.x & 0xffff0000u),
              __uint_as_float(w.y << 16), __uint_as_float(w.y & 0xffff0000u)};
  }
};
template <>
struct Raw4<SOPHIA_DTYPE_F32> {
  f4 w;
  __device__ __forceinline__ void load(const void *base, int64_t idx) {
    w = __builtin_nontemporal_load(reinterpret_cast<const f4 *>(static_cast<const float *>(base) + idx));
  }
  __device__ __forceinline__ f4 get() const { return w; }
};

// Bases of the swizzled [128 channel][64 row] bf16 tiles for the channels a
// lane owns (ch = 32 ks + 16 hf + 4 gq + j): swz(ch, row) = base[j] +
// 64 * (32 ks + 16 hf), since adding a multiple of 8 to ch leaves ch & 7 and
// the swizzle unchanged.  Stores then use compile-time offsets.
struct SwzBases {
  int b[4];
};
__device__ __forceinline__ SwzBases swz_bases(int gq, int row) {
  SwzBases s;
#pragma unroll
  for (int j = 0; j < 4; ++j) s.b[j] = swz(4 * gq + j, row);
  return s;
}

// Step 4 of the intra kernel for sub-block W (a compile-time wave index, so
// the products of sub-block totals below need no selects).  Per channel, with
// Gloc the within-sub-block cumulative log-decay and E_i = e^{tot_i}:
// a = e^{Gloc} (<= 1), b = e^{-Gloc} (<= e^80), kd = b E_W (<= 1),
// eref = e^{ref_W} = prod_{i<W} E_i, etail = e^{G_C - ref_{W+1}} = prod_{i>W} E_i.
// All products are of factors <= 1, so they can only underflow where the true
// value is below 2^-126.
template <int W, bool BWD>
__device__ __forceinline__ void intra_scaled_operands(
    const float (&qv)[32], const float (&kv)[32], const float (&gv)[32], float bt,
    const float *s_E, uint16_t *sKD, uint16_t *sKb, uint8_t *rec, const SwzBases &sb, int l,
    int lr, int gq, bf8 (&QSf)[4], bf8 (&KSf)[4], u4 (&kt_bits)[4], f4 &aqk_d, f4 &akk_d,
    uint8_t *brec, u4 (&qe_bits)[4]) {
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
    float qa[8], ka[8], kb[8], kd[8], kd1[8], kd2[8], kbar[8], qe[8], kt[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int e = 8 * ks + i;
      const f4 E = *reinterpret_cast<const f4 *>(&s_E[perm_k(ks, gq, i) * 4]);
      const float a = __builtin_amdgcn_exp2f(gv[e]);
      const float b = __builtin_amdgcn_exp2f(-gv[e]);
      float eref = 1.f, etl = 1.f;
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        if (m < W) eref *= E[m];
        if (m > W) etl *= E[m];
      }
      qa[i] = qv[e] * a;
      ka[i] = kv[e] * a;
      kb[i] = kv[e] * b;
      kd[i] = kb[i] * E[W];
      if constexpr (W < 2) kd1[i] = kd[i] * E[W + 1];   // for query block W+2
      if constexpr (W < 1) kd2[i] = kd1[i] * E[W + 2];  // for query block W+3
      kbar[i] = kd[i] * etl;
      qe[i] = qa[i] * eref;                             // Q e^G
      kt[i] = (bt * eref) * ka[i];                      // beta K e^G
    }
    QSf[ks] = pack8(qa);
    KSf[ks] = pack8(ka);
    const bf8 kbf = pack8(kb);
    aqk_d = mfma32(QSf[ks], kbf, aqk_d);
    akk_d = mfma32(KSf[ks], kbf, akk_d);
    kt_bits[ks] = bf8_to_bits(pack8(kt));
#pragma unroll
    for (int i = 0; i < 8; ++i)
      sKb[sb.b[i & 3] + 64 * (32 * ks + 16 * (i >> 2))] = f32_to_bf16_bits(kbar[i]);
    // Q e^G goes straight to the workspace in A-operand order (mb = W); the
    // backward's forward-state scan forms no O and reads no Q e^G.
    if constexpr (!BWD) *reinterpret_cast<u4 *>(rec + kOffQ + ((W * 4 + ks) * 64 + l) * 16) = bf8_to_bits(pack8(qe));
    if constexpr (BWD) {
      // Kbar in A-operand order (m = rows); Q e^G kept (bf16) for Qg^T, which
      // is transposed through LDS at the end of the item.
      *reinterpret_cast<u4 *>(brec + kBOffKbar + ((W * 4 + ks) * 64 + l) * 16) = bf8_to_bits(pack8(kbar));
      qe_bits[ks] = bf8_to_bits(pack8(qe));
    }
    // Key-side rows of this block for the later query blocks, row-major bf16.
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
      const int col = 32 * ks + 16 * hf + 4 * gq;
      const int i0 = 4 * hf;
      if constexpr (W < 3)
        *reinterpret_cast<u2 *>(&sKD[(kd_slot(W, 0) * 16 + lr) * kLdKD + col]) =
            u2{pack_bf16x2(kd[i0], kd[i0 + 1]), pack_bf16x2(kd[i0 + 2], kd[i0 + 3])};
      if constexpr (W < 2)
        *reinterpret_cast<u2 *>(&sKD[(kd_slot(W, 1) * 16 + lr) * kLdKD + col]) =
            u2{pack_bf16x2(kd1[i0], kd1[i0 + 1]), pack_bf16x2(kd1[i0 + 2], kd1[i0 + 3])};
      if constexpr (W < 1)
        *reinterpret_cast<u2 *>(&sKD[(kd_slot(W, 2) * 16 + lr) * kLdKD + col]) =
            u2{pack_bf16x2(kd2[i0], kd2[i0 + 1]), pack_bf16x2(kd2[i0 + 2], kd2[i0 + 3])};
    }
  }
}

// ---- fused ShortConv (kda_chunk_conv_intra_kernel) ----------------------------
// q, k, v arrive as the rows before the conv (whole lines in LDS: q in region
// A, k in C, v at stage_v; row r of wave w's 16 rows, 16-byte chunk j at chunk
// position j ^ r).  Lane l < 48 of wave w convolves chunk l & 15 (8 channels)
// of tensor l >> 4 (q, k, v) over the wave's 16 rows, in place, exactly as
// short_conv_fwd_kernel does: acc = sum_j taps[j] x[t - 3 + j] by fused
// multiply-adds from j = 0, y = acc sigmoid(acc), rounded to bf16.  The 3 rows
// before a wave's rows: rows 13..15 of wave w - 1 (read before any wave
// overwrites them); for wave 0 the 3 rows before the chunk, or, in the
// sequence's first chunk, its history (rounded to bf16, as the separate conv
// reads it) or zeros.
struct ConvPre {
  f4 taps[8];   // taps of channel 8j + i
  u4 halo[6];   // wave 0: the 3 rows before the chunk (bf16, halo[0..2]) or the fp32 history [8][3]
};

__device__ __forceinline__ size_t conv_region(int tn, int w) {
  return tn == 0 ? kSmA + w * 4096 : (tn == 1 ? kSmC + w * 4096 : stage_v(w));
}

__device__ __forceinline__ void unpack_bf16x8(u4 v, float (&x)[8]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    x[2 * i] = __uint_as_float(v[i] << 16);
    x[2 * i + 1] = __uint_as_float(v[i] & 0xffff0000u);
  }
}

// Issues the loads of the taps and of wave 0's 3 rows before the chunk.
__device__ __forceinline__ ConvPre conv_issue(const IntraArgs &p, int s, bool first_chunk, int h, int w, int l,
                                              int64_t t0) {
  ConvPre cp;
  const int tn = l >> 4, j = l & 15;
#pragma unroll
  for (int i = 0; i < 6; ++i) cp.halo[i] = u4{0u, 0u, 0u, 0u};
  if (l < 48) {
    const int64_t ch = (static_cast<int64_t>(tn) * p.num_heads + h) * kD + 8 * j;
    const f4 *tw = reinterpret_cast<const f4 *>(p.conv_w + ch * 4);
#pragma unroll
    for (int i = 0; i < 8; ++i) cp.taps[i] = tw[i];
    if (w == 0) {
      if (!first_chunk) {
        const uint16_t *x = static_cast<const uint16_t *>(tn == 0 ? p.q : (tn == 1 ? p.k : p.v));
#pragma unroll
        for (int r = 0; r < 3; ++r)
          cp.halo[r] = *reinterpret_cast<const u4 *>(x + (t0 - 3 + r) * p.qkv_stride + h * kD + 8 * j);
      } else {
        const int slot = p.conv_slots ? p.conv_slots[s] : s;
        if (p.conv_read && p.conv_state && slot >= 0 && slot < p.conv_n_slots) {
          const u4 *hp = reinterpret_cast<const u4 *>(
              p.conv_state + (static_cast<int64_t>(slot) * 3 * p.num_heads * kD + ch) * 3);
#pragma unroll
          for (int i = 0; i < 6; ++i) cp.halo[i] = hp[i];
        }
      }
    }
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) cp.taps[i] = f4{0.f, 0.f, 0.f, 0.f};
  }
  return cp;
}

// Convolves the wave's rows in LDS (after every wave's line copies landed).
__device__ __forceinline__ void conv_apply(const ConvPre &cp, bool first_chunk, int w, int l, uint8_t *smem) {
  const int tn = l >> 4, j = l & 15;
  const bool on = l < 48;
  float win[3][8];
  __builtin_amdgcn_s_waitcnt(0);  // this wave's line copies (every load so far) have landed
  lds_barrier();                  // ... and every wave's
  if (on) {
    if (w > 0) {
      const uint8_t *prev = smem + conv_region(tn, w - 1);
#pragma unroll
      for (int k = 0; k < 3; ++k) {
        const int r = 13 + k;
        unpack_bf16x8(*reinterpret_cast<const u4 *>(prev + r * 256 + ((j ^ r) << 4)), win[k]);
      }
    } else if (!first_chunk) {
#pragma unroll
      for (int k = 0; k < 3; ++k) unpack_bf16x8(cp.halo[k], win[k]);
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int k = 0; k < 3; ++k) {
          const int e = 3 * i + k;  // history [channel i][k]
          win[k][i] = bf16_bits_to_f32(f32_to_bf16_bits(__uint_as_float(cp.halo[e >> 2][e & 3])));
        }
    }
  }
  lds_barrier();  // every window is read before any row is overwritten
  if (!on) return;
  uint8_t *reg = smem + conv_region(tn, w);
#pragma unroll
  for (int half = 0; half < 2; ++half) {
    u4 rows[8];
#pragma unroll
    for (int rr = 0; rr < 8; ++rr) {
      const int r = 8 * half + rr;
      rows[rr] = *reinterpret_cast<const u4 *>(reg + r * 256 + ((j ^ r) << 4));
    }
#pragma unroll
    for (int rr = 0; rr < 8; ++rr) {
      const int r = 8 * half + rr;
      float x[8], y[8];
      unpack_bf16x8(rows[rr], x);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        float acc = 0.f;
        acc = fmaf(cp.taps[i][0], win[0][i], acc);
        acc = fmaf(cp.taps[i][1], win[1][i], acc);
        acc = fmaf(cp.taps[i][2], win[2][i], acc);
        acc = fmaf(cp.taps[i][3], x[i], acc);
        y[i] = acc * sigmoid_f(acc);
        win[0][i] = win[1][i];
        win[1][i] = win[2][i];
        win[2][i] = x[i];
      }
      *reinterpret_cast<u4 *>(reg + r * 256 + ((j ^ r) << 4)) =
          u4{pack_bf16x2(y[0], y[1]), pack_bf16x2(y[2], y[3]), pack_bf16x2(y[4], y[5]), pack_bf16x2(y[6], y[7])};
    }
  }
}

// One (chunk c, head h) of the intra phase on 256 threads (tid 0..255, four
// wavefronts) with kSmIntra bytes of LDS at smem; writes the record at rec.
// Every barrier inside is a work-group barrier: a work-group running two
// items at once runs them in lock step.
// BWD: the backward's instantiation, which also writes the backward record,
// T and P of the item (IntraArgs::brec / tpmat), in the same LDS.
// CONV: q, k, v are the rows before the fused ShortConv (bf16 whole lines only).
template <int QKV_DT, int G_DT, bool GATE, bool BWD = false, bool CONV = false>
__device__ __forceinline__ void intra_item(const IntraArgs &p, int c, int s, int first, int h, uint8_t *smem,
                                           int tid, uint8_t *rec) {
  static_assert(!CONV || (QKV_DT == SOPHIA_DTYPE_BF16 && !BWD), "the fused conv takes bf16 lines, forward only");
  const size_t item = static_cast<size_t>(c) * p.num_heads + h;
  uint8_t *brec = BWD ? p.brec + item * kBwdRecBytes : nullptr;
  uint16_t *sQt = reinterpret_cast<uint16_t *>(smem + kSmA);   // backward, at the end: Q e^G transposed
  uint16_t *sDo = reinterpret_cast<uint16_t *>(smem + kSmB);   // backward, at the end: dO transposed
  float *s_E = reinterpret_cast<float *>(smem + kSmE);
  uint16_t *sKD = reinterpret_cast<uint16_t *>(smem + kSmA);
  uint16_t *sKt = reinterpret_cast<uint16_t *>(smem + kSmA);
  uint16_t *sV = reinterpret_cast<uint16_t *>(smem + kSmB);
  uint16_t *sKb = reinterpret_cast<uint16_t *>(smem + kSmC);
  float *sT = reinterpret_cast<float *>(smem + kSmC);
  uint16_t *sQK = reinterpret_cast<uint16_t *>(smem + kSmD);

  const int64_t seq_a = iclamp64(p.cu[s], 0, p.total);
  const int64_t seq_b = iclamp64(p.cu[s + 1], seq_a, p.total);
  const int64_t t0 = seq_a + static_cast<int64_t>(c - first) * kC;
  const int len = static_cast<int>(imin64(kC, seq_b - t0));

  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave = 16-row sub-block (uniform)
  const int l = tid & 63;
  const int lr = l & 15;         // row within the sub-block
  const int gq = l >> 4;         // lane group
  const int row = 16 * w + lr;   // chunk row of this lane
  const bool valid = row < len;
  const int64_t tok = t0 + row;
  const SwzBases sb = swz_bases(gq, row);

  // ---- 1. load q, k, g (32 channels per lane, 16x16x32 operand order), v, beta.
  // Slot (ks, e) of a lane holds channel perm_k(ks, gq, e).  Every global load
  // of the block is issued before the first use, so the block pays one memory
  // round trip.  Rows past the end of the sequence load row t0 (always inside
  // it) and are masked afterwards through scale factors: beta and the q/k
  // norm scales become 0 and g is multiplied by 0 (no per-element branch).
  float qv[32], kv[32], gv[32];
  float bt;
  const float vmask = valid ? 1.f : 0.f;
  {
    const int64_t ltok = valid ? tok : t0;
    const int64_t qrow = ltok * p.qkv_stride + static_cast<int64_t>(h) * kD;
    const int64_t grow = ltok * p.g_stride + static_cast<int64_t>(h) * kD;
    // Gate parameters and beta are issued first (memory returns in issue
    // order); beta is kept as raw bits until after the loads: converting it
    // inside the dtype branch would make the wave wait right there.
    float hs = 1.f;
    f4 rb[8];
    if constexpr (GATE) {
      hs = p.A_log[h];
#pragma unroll
      for (int i = 0; i < 8; ++i)
        rb[i] = *reinterpret_cast<const f4 *>(p.dt_bias + h * kD + 32 * (i >> 1) + 16 * (i & 1) + 4 * gq);
    }
    uint32_t braw;
    const int64_t bidx = ltok * p.beta_stride + h;
    if (p.beta_dtype == SOPHIA_DTYPE_BF16)
      braw = static_cast<const uint16_t *>(p.beta)[bidx];
    else
      braw = static_cast<const uint32_t *>(p.beta)[bidx];
    Raw4<QKV_DT> rq[8], rk[8], rv[8];
    Raw4<G_DT> rg[8];
    bool lines = false;
    if constexpr (QKV_DT == SOPHIA_DTYPE_BF16) lines = CONV || p.qkv_lines != 0;
    ConvPre cpre;
    if constexpr (CONV) cpre = conv_issue(p, s, c == first, h, w, l, t0);
    if (lines) {
      // Whole cache lines: each wave copies its 16 rows of q, k, v (256 B per
      // row and head) straight into LDS, four rows per instruction, 16-byte
      // chunk j of row r at chunk position j ^ r (conflict-free reads below).
      // The slots are read back after the loads of g below have been issued.
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const int r = 4 * t + (l >> 4);
        const int64_t rt = 16 * w + r < len ? t0 + 16 * w + r : t0;
        const int64_t off = rt * p.qkv_stride + static_cast<int64_t>(h) * kD + 8 * ((l & 15) ^ r);
        const int dst = w * 4096 + t * 1024;
        __builtin_amdgcn_global_load_lds(static_cast<const uint16_t *>(p.q) + off, smem + kSmA + dst, 16, 0, 2);
        __builtin_amdgcn_global_load_lds(static_cast<const uint16_t *>(p.k) + off, smem + kSmC + dst, 16, 0, 2);
        __builtin_amdgcn_global_load_lds(static_cast<const uint16_t *>(p.v) + off, smem + stage_v(w) + t * 1024, 16,
                                         0, 2);
      }
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int ch = 32 * (i >> 1) + 16 * (i & 1) + 4 * gq;
        rq[i].load(p.q, qrow + ch);
        rk[i].load(p.k, qrow + ch);
        rv[i].load(p.v, qrow + ch);
      }
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) rg[i].load(p.g, grow + 32 * (i >> 1) + 16 * (i & 1) + 4 * gq);
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (CONV) conv_apply(cpre, c == first, w, l, smem);
    if constexpr (QKV_DT == SOPHIA_DTYPE_BF16) {
      if (lines) {
        // Slot i = 2 ks + a holds channels 32 ks + 16 a + 4 gq .. + 3: bytes
        // 8 (gq & 1) of chunk 4 ks + 2 a + gq / 2 of row lr.
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const int at = w * 4096 + lr * 256 + (((2 * i + (gq >> 1)) ^ lr) << 4) + 8 * (gq & 1);
          rq[i].w = *reinterpret_cast<const u2 *>(smem + kSmA + at);
          rk[i].w = *reinterpret_cast<const u2 *>(smem + kSmC + at);
          rv[i].w = *reinterpret_cast<const u2 *>(smem + stage_v(w) + (at - w * 4096));
        }
      }
    }
    bt = __uint_as_float(p.beta_dtype == SOPHIA_DTYPE_BF16 ? (braw << 16) : braw);
    if (p.flags & SOPHIA_KDA_BETA_SIGMOID) bt = fast_sigmoid(bt);
    bt *= vmask;
    if constexpr (GATE) hs = __expf(hs);
    // Log-decays are kept in base 2 (times log2 e) from here on, so that each
    // exponential below is one v_exp_f32.
    const float glb = (GATE ? p.lb * vmask : vmask) * kLog2e;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const f4 a = rq[i].get(), b = rk[i].get(), cc = rv[i].get(), d = rg[i].get();
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int e = 4 * i + j;
        qv[e] = a[j];
        kv[e] = b[j];
        if constexpr (GATE)
          gv[e] = glb * fast_sigmoid(hs * (d[j] + rb[i][j]));
        else
          gv[e] = glb * d[j];
        sV[sb.b[j] + 64 * (32 * (i >> 1) + 16 * (i & 1))] = f32_to_bf16_bits(bt * cc[j]);  // beta V^T
      }
    }
  }

  // ---- 2. l2 norms (a row is spread over the 4 lane groups)
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
    float qs = p.scale * vmask, ksc = vmask;
    if (p.flags & SOPHIA_KDA_QK_L2NORM) {
      qs *= __builtin_amdgcn_rcpf(fmaxf(sqrtf(sq), 1e-12f));
      ksc *= __builtin_amdgcn_rcpf(fmaxf(sqrtf(sk), 1e-12f));
    }
#pragma unroll
    for (int e = 0; e < 32; ++e) {
      qv[e] *= qs;
      kv[e] *= ksc;
    }
  }

  // ---- 3. within-sub-block cumulative log-decay (base 2); E[ch][i] = e^{tot_i}
#pragma unroll
  for (int e = 0; e < 32; ++e) gv[e] = row_scan16(gv[e]);
  if (lr == 15) {
#pragma unroll
    for (int e = 0; e < 32; ++e) s_E[perm_k(e >> 3, gq, e & 7) * 4 + w] = __builtin_amdgcn_exp2f(gv[e]);
  }
  lds_barrier();

  // ---- 4. scaled operands; diagonal 16x16 blocks of A_qk / A_kk
  bf8 QSf[4], KSf[4];           // query side (A operands), all key blocks
  u4 kt_bits[4];                // beta K e^G, bf16, operand order
  u4 qe_bits[4];                // backward only: Q e^G, bf16 (transposed at the end)
  f4 aqk_d = {0.f, 0.f, 0.f, 0.f}, akk_d = aqk_d;
  switch (w) {
    case 0: intra_scaled_operands<0, BWD>(qv, kv, gv, bt, s_E, sKD, sKb, rec, sb, l, lr, gq, QSf, KSf, kt_bits, aqk_d, akk_d, brec, qe_bits); break;
    case 1: intra_scaled_operands<1, BWD>(qv, kv, gv, bt, s_E, sKD, sKb, rec, sb, l, lr, gq, QSf, KSf, kt_bits, aqk_d, akk_d, brec, qe_bits); break;
    case 2: intra_scaled_operands<2, BWD>(qv, kv, gv, bt, s_E, sKD, sKb, rec, sb, l, lr, gq, QSf, KSf, kt_bits, aqk_d, akk_d, brec, qe_bits); break;
    default: intra_scaled_operands<3, BWD>(qv, kv, gv, bt, s_E, sKD, sKb, rec, sb, l, lr, gq, QSf, KSf, kt_bits, aqk_d, akk_d, brec, qe_bits); break;
  }
  lds_barrier();

  // ---- 4b. Kbar^T fragments (m = channels 16mb + lr for mb = 2w, 2w+1,
  //          k = chunk rows perm_k(ks, gq, .)) to the workspace; region C is
  //          then free for A_kk.
#pragma unroll
  for (int mi = 0; mi < 2; ++mi) {
    const int mb = 2 * w + mi;
    const int ch = 16 * mb + lr;
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const int r0 = 32 * ks + 4 * gq;
      const u2 lo = *reinterpret_cast<const u2 *>(&sKb[swz(ch, r0)]);
      const u2 hi = *reinterpret_cast<const u2 *>(&sKb[swz(ch, r0 + 16)]);
      *reinterpret_cast<u4 *>(rec + kOffKt + ((mb * 2 + ks) * 64 + l) * 16) = u4{lo.x, lo.y, hi.x, hi.y};
    }
  }
  lds_barrier();

  // ---- 5. off-diagonal blocks: key block ib < w uses copy v = w-1-ib of
  // its key-side rows (already scaled by prod_{ib<i<w} E_i).
  {
    float brow[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) brow[e] = __shfl(bt, 4 * gq + e, 64);
#pragma unroll
    for (int ib = 0; ib < 4; ++ib) {
      f4 aqk = {0.f, 0.f, 0.f, 0.f}, akk = aqk;
      if (ib == w) {
        aqk = aqk_d;
        akk = akk_d;
      } else if (ib < w) {
        const uint16_t *base = &sKD[(kd_slot(ib, w - 1 - ib) * 16 + lr) * kLdKD + 4 * gq];
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
          const u2 lo = *reinterpret_cast<const u2 *>(base + 32 * ks);
          const u2 hi = *reinterpret_cast<const u2 *>(base + 32 * ks + 16);
          const bf8 bk = bits_to_bf8(u4{lo.x, lo.y, hi.x, hi.y});
          aqk = mfma32(QSf[ks], bk, aqk);
          akk = mfma32(KSf[ks], bk, akk);
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
      if constexpr (BWD) {
        // P[r][col] (col < r) at [col][r]: four consecutive r per lane.
        float *tp = p.tpmat + item * (kC * kC) + col * kC + 16 * w + 4 * gq;
        if (ib < w) {
          *reinterpret_cast<f4 *>(tp) = akk;
        } else if (ib == w) {
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (col < 16 * w + 4 * gq + e) tp[e] = akk[e];
        }
      }
    }
  }
  lds_barrier();

  // ---- 6. T = (I + A_kk)^-1 in fp32.  Diagonal 16x16 blocks D_i by forward
  // substitution (one wave each), then the off-diagonal blocks.
  {
    float x[16];
    if (l < 16) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        float acc = (r == l) ? 1.f : 0.f;
#pragma unroll
        for (int j = 0; j < r; ++j) acc = fmaf(-sT[(16 * w + r) * kLdT + 16 * w + j], x[j], acc);
        x[r] = acc;
      }
    }
    // Each wave reads and rewrites only its own diagonal block.
    if (l < 16) {
#pragma unroll
      for (int r = 0; r < 16; ++r) sT[(16 * w + r) * kLdT + 16 * w + l] = x[r];
    }
    lds_barrier();
    // Off-diagonal blocks by sub-diagonal level d on fp32 MFMA:
    //   X_{i,i-d} = -D_i sum_{k=i-d}^{i-1} L_{i,k} X_{k,i-d},  X_{k,k} = D_k.
    // Wave i forms block row i.  Its L_{i,k} are read (as A operands) before
    // any X overwrites them; every other block it reads was written at a lower
    // level, before the barrier that ends that level.  A 16-deep product is
    // four 16x16x4 steps; step s of lane group g covers column 4g + s.
    const int g4 = 4 * gq;
    f4 Lrow[3], Dw;
#pragma unroll
    for (int k = 0; k < 3; ++k)
      Lrow[k] = *reinterpret_cast<const f4 *>(&sT[(16 * w + lr) * kLdT + 16 * k + g4]);
    Dw = *reinterpret_cast<const f4 *>(&sT[(16 * w + lr) * kLdT + 16 * w + g4]);
#pragma unroll
    for (int d = 1; d < 4; ++d) {
      if (w >= d) {
        const int j = w - d;
        f4 y = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int k = 0; k < 3; ++k) {
          if (k >= j && k < w) {
            float bx[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) bx[i] = sT[(16 * k + g4 + i) * kLdT + 16 * j + lr];
#pragma unroll
            for (int i = 0; i < 4; ++i) y = mfma_f32x4(Lrow[k][i], bx[i], y);
          }
        }
        f4 x = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int i = 0; i < 4; ++i) x = mfma_f32x4(Dw[i], y[i], x);
#pragma unroll
        for (int i = 0; i < 4; ++i) sT[(16 * w + g4 + i) * kLdT + 16 * j + lr] = -x[i];
      }
      lds_barrier();
    }
  }

  // ---- 7. beta K e^G, transposed, into region A (its scratch reads ended
  //         at the last barrier of the solve).
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
    const u4 kw = kt_bits[ks];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t kword = kw[i >> 1];
      sKt[sb.b[i & 3] + 64 * (32 * ks + 16 * (i >> 2))] =
          static_cast<uint16_t>((i & 1) ? (kword >> 16) : (kword & 0xffffu));
    }
  }
  lds_barrier();

  // ---- 8. Ut = T (beta V) for rows 16w .. 16w+15, and W^T = (beta K e^G)^T T^T
  //         for channels 32w .. 32w+31 and all 64 rows.  A C tile of W^T (rows =
  //         channels 16mb + 4gq + e, column = chunk row 16nb + lr), paired with the
  //         tile of channel block mb + 1, is the A-operand fragment of W for row
  //         block nb and K-step mb / 2: -W goes to the workspace from registers.
  //         Row r of T is zero past column r (lower triangular).
  const auto t_frag = [&](int row, int col0) {
    const f4 t0v = *reinterpret_cast<const f4 *>(&sT[row * kLdT + col0]);
    const f4 t1v = *reinterpret_cast<const f4 *>(&sT[row * kLdT + col0 + 4]);
    float ta[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      ta[i] = t0v[i];
      ta[4 + i] = t1v[i];
    }
    return pack8(ta);
  };
  f4 accU[8];
#pragma unroll
  for (int nt = 0; nt < 8; ++nt) accU[nt] = f4{0.f, 0.f, 0.f, 0.f};
  {
    const int nks = (w < 2) ? 1 : 2;
    for (int ks = 0; ks < nks; ++ks) {
      const bf8 af = t_frag(16 * w + lr, 32 * ks + 8 * gq);
#pragma unroll
      for (int nt = 0; nt < 8; ++nt) {
        const bf8 bv = bits_to_bf8(*reinterpret_cast<const u4 *>(&sV[swz(16 * nt + lr, 32 * ks + 8 * gq)]));
        accU[nt] = mfma32(af, bv, accU[nt]);
      }
    }
  }
  f4 accW[2][4];  // [channel block 2w + mi][row block nb]
  {
    bf8 kta[2][2];  // (beta K e^G)^T, A operand: m = channels 16(2w + mi) + lr
#pragma unroll
    for (int mi = 0; mi < 2; ++mi)
#pragma unroll
      for (int ks = 0; ks < 2; ++ks)
        kta[mi][ks] = bits_to_bf8(*reinterpret_cast<const u4 *>(&sKt[swz(16 * (2 * w + mi) + lr, 32 * ks + 8 * gq)]));
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) {
      accW[0][nb] = accW[1][nb] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < (nb < 2 ? 1 : 2); ++ks) {
        const bf8 tb = t_frag(16 * nb + lr, 32 * ks + 8 * gq);
#pragma unroll
        for (int mi = 0; mi < 2; ++mi) accW[mi][nb] = mfma32(kta[mi][ks], tb, accW[mi][nb]);
      }
    }
    if constexpr (BWD) {
      // W itself (the same fragments with the operands swapped): C tiles of
      // rows 16nb + 4gq + e and channel 16(2w + mi) + lr.  The tiles of row
      // blocks 2ks and 2ks + 1 are the two halves of the -W^T A operand of
      // K-step ks (k = chunk rows perm_k(ks, gq, .)).
#pragma unroll
      for (int mi = 0; mi < 2; ++mi) {
        f4 wt[4];
#pragma unroll
        for (int nb = 0; nb < 4; ++nb) {
          wt[nb] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int ks = 0; ks < (nb < 2 ? 1 : 2); ++ks)
            wt[nb] = mfma32(t_frag(16 * nb + lr, 32 * ks + 8 * gq), kta[mi][ks], wt[nb]);
        }
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
          float t[8];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            t[e] = -wt[2 * ks][e];
            t[4 + e] = -wt[2 * ks + 1][e];
          }
          *reinterpret_cast<u4 *>(brec + kBOffWt + (((2 * w + mi) * 2 + ks) * 64 + l) * 16) = bf8_to_bits(pack8(t));
        }
      }
    }
  }

  // ---- 9. Ut in C-tile order and -W as A-operand fragments (m = chunk rows
  //         16nb + lr, k = channels perm_k(w, gq, .)) to the workspace; e^{G_C}.
#pragma unroll
  for (int nt = 0; nt < 8; ++nt)
    *reinterpret_cast<u2 *>(rec + kOffU + ((w * 8 + nt) * 64 + l) * 8) = pack4_bf16(accU[nt]);
#pragma unroll
  for (int nb = 0; nb < 4; ++nb) {
    float t[8];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      t[e] = -accW[0][nb][e];
      t[4 + e] = -accW[1][nb][e];
    }
    *reinterpret_cast<u4 *>(rec + kOffW + ((nb * 4 + w) * 64 + l) * 16) = bf8_to_bits(pack8(t));
  }
  if (tid < kD) {
    const f4 E = *reinterpret_cast<const f4 *>(&s_E[tid * 4]);
    reinterpret_cast<float *>(rec + kOffG)[tid] = E[0] * E[1] * E[2] * E[3];
  }
  if constexpr (BWD) {
    // T, its lower triangle (the strict upper one holds P): thread t copies
    // row t / 4, 16 columns.
    const int r = tid >> 2, c0 = 16 * (tid & 3);
    float *tp = p.tpmat + item * (kC * kC) + r * kC;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = c0 + 4 * i;
      const f4 tv = *reinterpret_cast<const f4 *>(&sT[r * kLdT + c]);
      if (c + 3 <= r) {
        *reinterpret_cast<f4 *>(tp + c) = tv;
      } else if (c <= r) {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (c + e <= r) tp[c + e] = tv[e];
      }
    }
    // A_qk^T fragments: m = chunk rows j = 16w + lr, k = rows i perm_k(ks, gq, .).
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      uint32_t wd[4];
#pragma unroll
      for (int e = 0; e < 8; e += 2) {
        const uint32_t a = sQK[perm_k(ks, gq, e) * kLdQK + 16 * w + lr];
        const uint32_t b = sQK[perm_k(ks, gq, e + 1) * kLdQK + 16 * w + lr];
        wd[e >> 1] = a | (b << 16);
      }
      *reinterpret_cast<u4 *>(brec + kBOffAt + ((w * 2 + ks) * 64 + l) * 16) = u4{wd[0], wd[1], wd[2], wd[3]};
    }
  }

  // ---- 10. A_qk fragments from LDS to the workspace (not for the backward's
  // forward-state scan, which forms no O)
  // A_qk: m = chunk rows 16w + lr, k = chunk rows perm_k(ks, gq, .).  The
  // fragments of K-step 1 for rows 0..31 are zero (A_qk is lower
  // triangular): they are neither written nor read.
  if constexpr (BWD) {
    // Qg^T and dO as fragments of the backward record, transposed through
    // regions A and B (their last reads were in step 8): Q e^G from the
    // registers of step 4, dO rows loaded here (rows past the sequence end
    // are zero).
    const int64_t drow = (valid ? tok : t0) * p.do_stride + static_cast<int64_t>(h) * kD;
    f4 dov[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) dov[i] = load4(p.dout, drow + 32 * (i >> 1) + 16 * (i & 1) + 4 * gq, p.do_dtype);
    lds_barrier();
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const uint32_t qword = qe_bits[ks][i >> 1];
        sQt[sb.b[i & 3] + 64 * (32 * ks + 16 * (i >> 2))] =
            static_cast<uint16_t>((i & 1) ? (qword >> 16) : (qword & 0xffffu));
      }
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        sDo[sb.b[j] + 64 * (32 * (i >> 1) + 16 * (i & 1))] = f32_to_bf16_bits(vmask * dov[i][j]);
    lds_barrier();
#pragma unroll
    for (int mi = 0; mi < 2; ++mi) {
      const int mb = 2 * w + mi;
      const int ch = 16 * mb + lr;
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const int r0 = 32 * ks + 4 * gq;
        const u2 qlo = *reinterpret_cast<const u2 *>(&sQt[swz(ch, r0)]);
        const u2 qhi = *reinterpret_cast<const u2 *>(&sQt[swz(ch, r0 + 16)]);
        *reinterpret_cast<u4 *>(brec + kBOffQt + ((mb * 2 + ks) * 64 + l) * 16) = u4{qlo.x, qlo.y, qhi.x, qhi.y};
        // dO B operand of value-column tile nt = mb (k = the same chunk rows).
        const u2 dlo = *reinterpret_cast<const u2 *>(&sDo[swz(ch, r0)]);
        const u2 dhi = *reinterpret_cast<const u2 *>(&sDo[swz(ch, r0 + 16)]);
        *reinterpret_cast<u4 *>(brec + kBOffDo + ((ks * 8 + mb) * 64 + l) * 16) = u4{dlo.x, dlo.y, dhi.x, dhi.y};
      }
    }
    return;
  }
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) {
    if (ks == 1 && w < 2) break;
    const uint16_t *src = &sQK[(16 * w + lr) * kLdQK + 32 * ks + 4 * gq];
    const u2 lo = *reinterpret_cast<const u2 *>(src);
    const u2 hi = *reinterpret_cast<const u2 *>(src + 16);
    *reinterpret_cast<u4 *>(rec + kOffA + ((w * 2 + ks) * 64 + l) * 16) = u4{lo.x, lo.y, hi.x, hi.y};
  }
}

template <int QKV_DT, int G_DT, bool GATE>
__global__ __launch_bounds__(kThreads, 2) void kda_chunk_intra_kernel(IntraArgs p) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  // Head-fastest order: the heads of one chunk run together and read the
  // same token rows (measured 3-10 % faster than chunk-fastest; the scan that
  // follows also reads the records faster).  Chunks run last first (see above).
  const int h = static_cast<int>(blockIdx.x % static_cast<unsigned>(p.num_heads));
  const int c = static_cast<int>(p.max_ch - 1) - static_cast<int>(blockIdx.x / static_cast<unsigned>(p.num_heads));
  if (c < 0) return;
  int s, first;
  chunk_of(p.cu, p.n_seqs, p.total, c, s, first);
  if (s >= p.n_seqs) return;  // past the last chunk (uniform over the work-group)
  intra_item<QKV_DT, G_DT, GATE>(p, c, s, first, h, smem, threadIdx.x,
                                 p.records + (static_cast<size_t>(c) * p.num_heads + h) * kRecBytes);
}

// The forward with the ShortConv of q, k, v fused in: q, k, v are bf16 rows
// before the conv (16-byte aligned, whole lines), IntraArgs::conv_* the taps
// and histories.  Items and records as kda_chunk_intra_kernel.
template <int G_DT, bool GATE>
__global__ __launch_bounds__(kThreads, 2) void kda_chunk_conv_intra_kernel(IntraArgs p) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int h = static_cast<int>(blockIdx.x % static_cast<unsigned>(p.num_heads));
  const int c = static_cast<int>(p.max_ch - 1) - static_cast<int>(blockIdx.x / static_cast<unsigned>(p.num_heads));
  if (c < 0) return;
  int s, first;
  chunk_of(p.cu, p.n_seqs, p.total, c, s, first);
  if (s >= p.n_seqs) return;
  intra_item<SOPHIA_DTYPE_BF16, G_DT, GATE, false, true>(
      p, c, s, first, h, smem, threadIdx.x, p.records + (static_cast<size_t>(c) * p.num_heads + h) * kRecBytes);
}

// New conv histories after kda_chunk_conv_intra_kernel has read the old ones:
// history[slot(s)][ch][0..2] <- the last 3 rows of cat(history (bf16-rounded,
// or zeros), x rows of sequence s), as short_conv_history_kernel writes them.
// One thread per (sequence = blockIdx.y, tensor, head, 8-channel chunk).
__global__ __launch_bounds__(256) void kda_conv_history_kernel(IntraArgs p) {
  const int t = blockIdx.x * 256 + threadIdx.x;
  const int s = blockIdx.y;
  const int per_tensor = p.num_heads * (kD / 8);
  if (t >= 3 * per_tensor || s >= p.n_seqs || !p.conv_state) return;
  const int slot = p.conv_slots ? p.conv_slots[s] : s;
  if (slot < 0 || slot >= p.conv_n_slots) return;
  const int tn = t / per_tensor, rem = t - tn * per_tensor;
  const int h = rem / (kD / 8), j = rem % (kD / 8);
  const int64_t start = iclamp64(p.cu[s], 0, p.total);
  const int64_t end = iclamp64(p.cu[s + 1], start, p.total);
  const uint16_t *x = static_cast<const uint16_t *>(tn == 0 ? p.q : (tn == 1 ? p.k : p.v));
  float *hist = p.conv_state +
                (static_cast<int64_t>(slot) * 3 * p.num_heads * kD + (static_cast<int64_t>(tn) * p.num_heads + h) * kD +
                 8 * j) * 3;
  float nh[8][3];
#pragma unroll
  for (int k = 0; k < 3; ++k) {
    const int64_t tau = end - 3 + k;
    if (tau >= start) {
      float v[8];
      unpack_bf16x8(*reinterpret_cast<const u4 *>(x + tau * p.qkv_stride + h * kD + 8 * j), v);
#pragma unroll
      for (int i = 0; i < 8; ++i) nh[i][k] = v[i];
    } else {
      const int idx = 3 + static_cast<int>(tau - start);
#pragma unroll
      for (int i = 0; i < 8; ++i)
        nh[i][k] = p.conv_read ? bf16_bits_to_f32(f32_to_bf16_bits(hist[i * 3 + idx])) : 0.f;
    }
  }
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int k = 0; k < 3; ++k) hist[i * 3 + k] = nh[i][k];
}

// The backward's instantiation: the same item, plus the backward record, T
// and P (two work-groups per CU, as the forward's).
template <int QKV_DT, int G_DT, bool GATE>
__global__ __launch_bounds__(kThreads, 2) void kda_chunk_intra_bwd_kernel(IntraArgs p) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int h = static_cast<int>(blockIdx.x % static_cast<unsigned>(p.num_heads));
  const int c = static_cast<int>(p.max_ch - 1) - static_cast<int>(blockIdx.x / static_cast<unsigned>(p.num_heads));
  if (c < 0) return;
  int s, first;
  chunk_of(p.cu, p.n_seqs, p.total, c, s, first);
  if (s >= p.n_seqs) return;
  intra_item<QKV_DT, G_DT, GATE, true>(p, c, s, first, h, smem, threadIdx.x,
                                       p.records + (static_cast<size_t>(c) * p.num_heads + h) * kRecBytes);
}

// ---- scan kernel -------------------------------------------------------------
// Batches of at most kOrderMax sequences whose offsets the host also holds are
// scanned longest sequence first.
struct ScanArgs {
  const int32_t *cu;
  int n_seqs;
  int64_t total;
  int num_heads;
  int64_t max_ch;
  const uint8_t *records;
  const float *h0;
  float *ht;
  int n_slots;
  const int32_t *slots;
  void *o;
  int64_t o_stride;
  void *trash;  // kTrashBytes of workspace: destination of rows past a sequence end
  // Sequence taken by the work-groups of rank r < kOrderMax: 4-bit field r
  // (r itself from kOrderMax on).  Packed into one argument and extracted
  // arithmetically: an indexed load here (even a scalar one) changes the
  // registers the compiler gives the rings, and its wait counts drain them.
  uint64_t order_bits;
  // Launch plan: up to kMaxClasses classes of consecutive ranks.  Class c
  // owns work-groups [cls_block[c], cls_block[c + 1]) and ranks [cls_rank[c],
  // cls_rank[c + 1]); each of its (sequence, head) pairs runs on
  // cls_splits[c] work-groups of 128 / cls_splits[c] value columns.  The
  // fields are read by name and selected with compares (see above).
  int n_cls;
  int cls_block0, cls_block1, cls_block2, cls_block3;
  int cls_rank0, cls_rank1, cls_rank2, cls_rank3, cls_rank4;
  int cls_splits0, cls_splits1, cls_splits2, cls_splits3;
};

// ---- scan kernel: two roles per work-group ----------------------------------
// Wavefronts 0..3 ("U/O" role) own chunk rows 16w..16w+15: U = Ut - W S and
// O = (Q e^G) S + A_qk U.  Wavefronts 4..7 ("state" role) own state rows
// 32sw..32sw+31 (sw = wave - 4) and the fp32 state: S <- Diag(e^{G_C}) S +
// Kbar^T U.  Per chunk: the state waves publish S (bf16 B operand) -> barrier ->
// the U/O waves form U and publish it -> barrier -> the state waves update S
// while the U/O waves finish O and store it.  Each role streams only its own
// record fragments, through a ring of register buffers of its own.
constexpr int kScanThreads = 512;
// What a scan work-group computes.
//  kModeRun:      the chain's outputs O and its final state.
//  kModeComposeM: the linear part M of the chain's map S -> M S + B (start
//                 from S = I, no Ut, no O); fin receives M.
//  kModeComposeB: its affine part B (start from S = 0, no O); fin receives B.
constexpr int kModeRun = 0;
constexpr int kModeComposeM = 1;
constexpr int kModeComposeB = 2;
// Ring depths (record buffers in flight): the U/O buffers grow with the
// number of value-column tiles, so the widest work-group keeps two.
template <int NT>
constexpr int ring_uo() { return NT >= 8 ? 2 : 3; }
constexpr int kRingS = 4;

template <int NT>
struct UOFrags {
  u4 wn[4];   // -W, A operand, m = rows 16w.., k = channels perm_k(ks, gq, .)
  u4 qb[4];   // Q e^G, A operand
  u4 aq[2];   // A_qk, A operand, k = chunk rows perm_k(ks, gq, .)
  u2 ut[NT];  // Ut, C tile (rows 16w + 4gq + e, column 16(nt0 + nt) + lr), bf16
};

struct SFrags {
  u4 kt[2][2];  // Kbar^T, A operand, m = channels 16(2sw + mi) + lr, ks 0..1
  f4 gm[2];     // e^{G_C} of state rows 32sw + 16mi + 4gq + e
};

// The operands used before the U barrier (-W, Q e^G, Ut) ...
template <int NT, int MODE = kModeRun>
__device__ __forceinline__ void load_uo_main(UOFrags<NT> &f, const uint8_t *rec, int w, int l, int nt0) {
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
    f.wn[ks] = *reinterpret_cast<const u4 *>(rec + kOffW + ((w * 4 + ks) * 64 + l) * 16);
    if constexpr (MODE == kModeRun)
      f.qb[ks] = *reinterpret_cast<const u4 *>(rec + kOffQ + ((w * 4 + ks) * 64 + l) * 16);
  }
  if constexpr (MODE != kModeComposeM) {
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
      f.ut[nt] = *reinterpret_cast<const u2 *>(rec + kOffU + ((w * 8 + nt0 + nt) * 64 + l) * 8);
  }
}
// ... and A_qk, used after it.  Rows 0..31 (w < 2) use K-step 0 only: their
// K-step-1 fragment is not in the record, so that load re-reads K-step 0
// (same lines, unused) instead of sitting under a branch.
template <int NT>
__device__ __forceinline__ void load_uo_aq(UOFrags<NT> &f, const uint8_t *rec, int w, int l) {
  f.aq[0] = *reinterpret_cast<const u4 *>(rec + kOffA + ((w * 2) * 64 + l) * 16);
  f.aq[1] = *reinterpret_cast<const u4 *>(rec + kOffA + ((w * 2 + (w >= 2 ? 1 : 0)) * 64 + l) * 16);
}

__device__ __forceinline__ void load_s(SFrags &f, const uint8_t *rec, int sw, int l, int gq) {
#pragma unroll
  for (int mi = 0; mi < 2; ++mi)
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
      f.kt[mi][ks] = *reinterpret_cast<const u4 *>(rec + kOffKt + (((2 * sw + mi) * 2 + ks) * 64 + l) * 16);
  const float *gam = reinterpret_cast<const float *>(rec + kOffG);
#pragma unroll
  for (int mi = 0; mi < 2; ++mi) f.gm[mi] = *reinterpret_cast<const f4 *>(&gam[32 * sw + 16 * mi + 4 * gq]);
}

// Makes the wave wait for the loads of a buffer here: an empty asm statement
// that reads every register of it.
template <int NT, int MODE = kModeRun>
__device__ __forceinline__ void touch(const UOFrags<NT> &f) {
  if constexpr (MODE == kModeRun) {
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) asm volatile("" ::"v"(f.wn[ks]), "v"(f.qb[ks]));
    asm volatile("" ::"v"(f.aq[0]), "v"(f.aq[1]));
  } else {
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) asm volatile("" ::"v"(f.wn[ks]));
  }
  if constexpr (MODE != kModeComposeM) {
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) asm volatile("" ::"v"(f.ut[nt]));
  }
}
__device__ __forceinline__ void touch(const SFrags &f) {
  asm volatile("" ::"v"(f.kt[0][0]), "v"(f.kt[0][1]), "v"(f.kt[1][0]), "v"(f.kt[1][1]));
  asm volatile("" ::"v"(f.gm[0]), "v"(f.gm[1]));
}

struct ScanGeom {
  int h, nt0, nchunks;
  int64_t tok_a, seq_b;
  const uint8_t *rec0;
  size_t rec_stride;
};

// Work of one scan work-group: a chain of consecutive chunks of one sequence
// (the whole sequence, or one segment of it).
struct Chain {
  int first;          // global number of the chain's first chunk
  int nchunks;        // chunks in the chain
  int64_t tok_a;      // first token of the chain
  int64_t seq_b;      // end of its sequence: rows at or past it go to the scratch rows
  const float *init;  // [128][128] fp32 state entering the chain, or NULL (zero)
  float *fin;         // where the state leaving the chain goes, or NULL
};


// One chunk of the U/O role, in two parts around the U barrier (two
// barriers in all).
//
// O is formed transposed: an A operand fragment of X (m x k) is, register for
// register, the B operand fragment of X^T, so swapping the operands of the
// products gives O^T = S^T (Q e^G)^T + U^T A_qk^T with the same fragments.  The
// O^T C tile puts 4 consecutive value columns of one token row in each lane:
// one 8-byte (bf16) or 16-byte (fp32) store per tile.
template <int NT, int MODE = kModeRun>
__device__ __forceinline__ void uo_pre(const UOFrags<NT> &f, f4 (&O)[NT], const uint8_t *sSb, uint8_t *sUb,
                                       int w, int l) {
  lds_barrier();  // S of this chunk is published
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    bf8 sb[4];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
      sb[ks] = bits_to_bf8(*reinterpret_cast<const u4 *>(sSb + ((ks * NT + nt) * 64 + l) * 16));
    f4 u = {0.f, 0.f, 0.f, 0.f};
    if constexpr (MODE != kModeComposeM) {
      const u2 uw = f.ut[nt];
      u = f4{__uint_as_float(uw.x << 16), __uint_as_float(uw.x & 0xffff0000u),
             __uint_as_float(uw.y << 16), __uint_as_float(uw.y & 0xffff0000u)};
    }
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) u = mfma32(bits_to_bf8(f.wn[ks]), sb[ks], u);
    // U rows 16w.. are half (w & 1) of K-step w / 2 of the U operand.
    *reinterpret_cast<u2 *>(sUb + (((w >> 1) * NT + nt) * 64 + l) * 16 + (w & 1) * 8) = pack4_bf16(u);
    if constexpr (MODE == kModeRun) {
      f4 o = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) o = mfma32(sb[ks], bits_to_bf8(f.qb[ks]), o);
      O[nt] = o;   // O^T tiles: value columns 16(nt0 + nt) + 4gq + e, token row 16w + lr
    }
  }
  lds_barrier();  // U is published
}

// Second part: O^T += U^T A_qk^T, then the stores.  Stores are never under a
// branch (a store under a branch makes the compiler drain the loads in flight
// at the join): rows past the end of the sequence go to a scratch row block
// in the workspace instead.
template <int NT, int O_DT>
__device__ __forceinline__ void uo_post(const ScanArgs &p, const ScanGeom &g, const UOFrags<NT> &f,
                                        f4 (&O)[NT], const uint8_t *sUb, int w, int l, int cc) {
  const int lr = l & 15, gq = l >> 4;
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const bf8 u0 = bits_to_bf8(*reinterpret_cast<const u4 *>(sUb + ((0 * NT + nt) * 64 + l) * 16));
    O[nt] = mfma32(u0, bits_to_bf8(f.aq[0]), O[nt]);
    if (w >= 2) {  // A_qk is lower triangular
      const bf8 u1 = bits_to_bf8(*reinterpret_cast<const u4 *>(sUb + ((1 * NT + nt) * 64 + l) * 16));
      O[nt] = mfma32(u1, bits_to_bf8(f.aq[1]), O[nt]);
    }
  }
  const int64_t tok0 = g.tok_a + static_cast<int64_t>(cc) * kC;
  const int r = 16 * w + lr;
  const bool row_ok = static_cast<int64_t>(r) < g.seq_b - tok0;
  const int64_t col = static_cast<int64_t>(g.h) * kD + 16 * g.nt0 + 4 * gq;
  const int64_t elem = row_ok ? (tok0 + r) * p.o_stride + col : static_cast<int64_t>(r) * kD + 16 * g.nt0 + 4 * gq;
  void *dst = row_ok ? p.o : p.trash;
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) store4(dst, elem + 16 * nt, O_DT, O[nt]);
}

// Publishes this wave's state rows as K-step sw of the bf16 B operand of S.
template <int NT>
__device__ __forceinline__ void publish_state(const f4 (&S)[2][NT], uint8_t *sSb, int sw, int l) {
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    float t[8];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      t[e] = S[0][nt][e];
      t[4 + e] = S[1][nt][e];
    }
    *reinterpret_cast<u4 *>(sSb + ((sw * NT + nt) * 64 + l) * 16) = bf8_to_bits(pack8(t));
  }
}

// Second half of a chunk of the state role: S <- Diag(e^{G_C}) S + Kbar^T U
// once U is published, then publish S for the next chunk.  (The first half is
// the barrier at which the U/O role picks S up.)
template <int NT>
__device__ __forceinline__ void state_update(const SFrags &f, f4 (&S)[2][NT], uint8_t *sSb,
                                             const uint8_t *sUb, int sw, int l) {
  lds_barrier();  // U published
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    bf8 ub[2];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
      ub[ks] = bits_to_bf8(*reinterpret_cast<const u4 *>(sUb + ((ks * NT + nt) * 64 + l) * 16));
#pragma unroll
    for (int mi = 0; mi < 2; ++mi) {
      f4 sv = S[mi][nt] * f.gm[mi];
      sv = mfma32(bits_to_bf8(f.kt[mi][0]), ub[0], sv);
      sv = mfma32(bits_to_bf8(f.kt[mi][1]), ub[1], sv);
      S[mi][nt] = sv;
    }
  }
  publish_state<NT>(S, sSb, sw, l);
}

// One work-group of 8 wavefronts per (sequence, head, NVB value columns).
// Record operands stream through per-role rings of register buffers, several
// chunks ahead.  A wave that issues loads faster than the CU's memory queue
// drains them stalls at the load, and a wave stalled there issues nothing
// else, so each role refills its ring in the part of the chunk where the
// other role is on the critical path: the state waves after the S barrier
// (while U is formed), the U/O waves after the U barrier (while S is
// updated).  The buffer of the next step is waited for right after the newest
// loads are issued (touch), where the wait can leave exactly those in flight;
// a wait placed by the compiler at a loop header would drain everything.  Loads are never
// under a branch (the compiler then drains every load at the join): past the
// last chunk they re-read the last chunk, unused.  The prologue issues the
// ring buffers strictly in order: the wait counts in the loop are the minimum
// over every path into it, so a prologue that interleaves the loads of two
// buffers makes every later step wait for its newest buffer too.
//
// scan_item: one chain (a sequence or a segment of one), head h and
// value-column slice `half` of the scan on 512 threads, with the S and U
// exchange buffers at sSb / sUb.  MODE selects what the chain computes.
template <int NVB, int O_DT, int MODE>
__device__ __forceinline__ void scan_item(const ScanArgs &p, const Chain &c, int h, int half, uint8_t *sSb,
                                          uint8_t *sUb) {
  constexpr int NT = NVB / 16;               // 16-column tiles per work-group
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l = tid & 63;
  const int lr = l & 15, gq = l >> 4;
  ScanGeom g;
  g.h = h;
  g.nt0 = half * NT;
  g.tok_a = c.tok_a;
  g.seq_b = c.seq_b;
  // Wave-uniform by construction; readfirstlane makes the compiler see it, so
  // that the per-chunk `live` tests below are scalar branches (a store under a
  // divergent branch makes the compiler drain the ring loads at the join).
  g.nchunks = __builtin_amdgcn_readfirstlane(c.nchunks);
  g.rec0 = p.records + (static_cast<size_t>(c.first) * p.num_heads + h) * kRecBytes;
  g.rec_stride = static_cast<size_t>(p.num_heads) * kRecBytes;
  const int nchunks = g.nchunks;
  const int last = nchunks - 1;

  if (wave < 4) {
    // ---- U/O role
    const int w = wave;
    if (nchunks <= 0) return;
    constexpr int R = ring_uo<NT>();
    UOFrags<NT> f[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const uint8_t *rec = g.rec0 + min(r, last) * g.rec_stride;
      load_uo_main<NT, MODE>(f[r], rec, w, l, g.nt0);
      if constexpr (MODE == kModeRun) load_uo_aq<NT>(f[r], rec, w, l);
      __builtin_amdgcn_sched_barrier(0);  // keep the ring order (see above)
    }
    touch<NT, MODE>(f[0]);
    for (int cc = 0; cc < nchunks; cc += R) {
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const bool live = cc + r < nchunks;
        const uint8_t *rec = g.rec0 + min(cc + r + R, last) * g.rec_stride;
        f4 O[NT];
        if (live) uo_pre<NT, MODE>(f[r], O, sSb, sUb, w, l);
        // Refill while the state role works: the loads may wait for memory
        // queue space here, off the critical path.
        load_uo_main<NT, MODE>(f[r], rec, w, l, g.nt0);
        if constexpr (MODE == kModeRun) {
          if (live) uo_post<NT, O_DT>(p, g, f[r], O, sUb, w, l, cc + r);
          load_uo_aq<NT>(f[r], rec, w, l);
        }
        touch<NT, MODE>(f[(r + 1) % R]);
      }
    }
    return;
  }

  // ---- state role: S tiles [mi 2][nt NT], rows 32sw + 16mi + 4gq + e,
  // column 16(nt0 + nt) + lr.
  const int sw = wave - 4;
  f4 S[2][NT];
#pragma unroll
  for (int mi = 0; mi < 2; ++mi)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      f4 v = {0.f, 0.f, 0.f, 0.f};
      if constexpr (MODE == kModeComposeM) {
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = (32 * sw + 16 * mi + 4 * gq + e == 16 * (g.nt0 + nt) + lr) ? 1.f : 0.f;
      } else if (c.init) {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          v[e] = c.init[static_cast<int64_t>(32 * sw + 16 * mi + 4 * gq + e) * kD + 16 * (g.nt0 + nt) + lr];
      }
      S[mi][nt] = v;
    }
  if (nchunks > 0) {
    publish_state<NT>(S, sSb, sw, l);
    // Buffer r holds chunk cc + r; after the S barrier of chunk c the buffer
    // of chunk c - 1 is refilled with chunk c + kRingS - 1 while the U/O role
    // forms U (the loads may wait for memory queue space there).
    SFrags f[kRingS];
#pragma unroll
    for (int r = 0; r < kRingS - 1; ++r) {
      load_s(f[r], g.rec0 + min(r, last) * g.rec_stride, sw, l, gq);
      __builtin_amdgcn_sched_barrier(0);
    }
    for (int cc = 0; cc < nchunks; cc += kRingS) {
#pragma unroll
      for (int r = 0; r < kRingS; ++r) {
        const bool live = cc + r < nchunks;
        if (live) lds_barrier();  // S published
        load_s(f[(r + kRingS - 1) % kRingS], g.rec0 + min(cc + r + kRingS - 1, last) * g.rec_stride, sw, l, gq);
        touch(f[r]);
        if (live) state_update<NT>(f[r], S, sSb, sUb, sw, l);
      }
    }
  }
  if (c.fin) {
#pragma unroll
    for (int mi = 0; mi < 2; ++mi)
#pragma unroll
      for (int nt = 0; nt < NT; ++nt)
#pragma unroll
        for (int e = 0; e < 4; ++e)
          c.fin[static_cast<int64_t>(32 * sw + 16 * mi + 4 * gq + e) * kD + 16 * (g.nt0 + nt) + lr] = S[mi][nt][e];
  }
}

// The chain of a whole sequence s, with its state slot.
__device__ __forceinline__ Chain sequence_chain(const ScanArgs &p, int s, int h) {
  Chain c;
  c.first = first_chunk(p.cu, p.n_seqs, p.total, s);
  c.tok_a = iclamp64(p.cu[s], 0, p.total);
  c.seq_b = iclamp64(p.cu[s + 1], c.tok_a, p.total);
  c.nchunks = static_cast<int>(imin64((c.seq_b - c.tok_a + kC - 1) / kC, p.max_ch - c.first));
  const int slot = p.slots ? p.slots[s] : s;
  const bool has_slot = slot >= 0 && slot < p.n_slots;  // else: zero start, nothing written
  const int64_t state_off = (static_cast<int64_t>(has_slot ? slot : 0) * p.num_heads + h) * kD * kD;
  c.init = p.h0 && has_slot ? p.h0 + state_off : nullptr;
  c.fin = p.ht && has_slot ? p.ht + state_off : nullptr;
  return c;
}

template <int O_DT>
__global__ __launch_bounds__(kScanThreads) void kda_chunk_scan_kernel(ScanArgs p) {
  // Exchange buffers sized for the widest slice (128 value columns).
  __shared__ __attribute__((aligned(16))) uint8_t sSb[4 * 8 * 64 * 16];   // S, [ks][nt][lane]
  __shared__ __attribute__((aligned(16))) uint8_t sUb[2 * 8 * 64 * 16];   // U, [ks][nt][lane]
  const int b = blockIdx.x;
  // Class of this work-group (uniform; scalar compares on kernel arguments).
  const bool c1 = p.n_cls > 1 && b >= p.cls_block1;
  const bool c2 = p.n_cls > 2 && b >= p.cls_block2;
  const bool c3 = p.n_cls > 3 && b >= p.cls_block3;
  const int start = c3 ? p.cls_block3 : c2 ? p.cls_block2 : c1 ? p.cls_block1 : p.cls_block0;
  const int rank_lo = c3 ? p.cls_rank3 : c2 ? p.cls_rank2 : c1 ? p.cls_rank1 : p.cls_rank0;
  const int rank_hi = c3 ? p.cls_rank4 : c2 ? p.cls_rank3 : c1 ? p.cls_rank2 : p.cls_rank1;
  const int splits = c3 ? p.cls_splits3 : c2 ? p.cls_splits2 : c1 ? p.cls_splits1 : p.cls_splits0;
  // XCD-aware order inside a class: the `splits` work-groups of one
  // (sequence, head) share the same local % 8, i.e. (classes start at
  // multiples of 8) the same XCD and L2, so they share record reads.
  const int local = b - start;
  const int group = local / (8 * splits);
  const int half = (local / 8) % splits;
  const int sh = group * 8 + (local % 8);
  const int h = sh % p.num_heads;
  const int rank = rank_lo + sh / p.num_heads;
  if (rank >= rank_hi || rank >= p.n_seqs) return;
  const int s = rank < kOrderMax ? static_cast<int>((p.order_bits >> (4 * rank)) & 15u) : rank;
  const Chain c = sequence_chain(p, s, h);
  switch (splits) {
    case 8: scan_item<16, O_DT, kModeRun>(p, c, h, half, sSb, sUb); break;
    case 4: scan_item<32, O_DT, kModeRun>(p, c, h, half, sSb, sUb); break;
    case 2: scan_item<64, O_DT, kModeRun>(p, c, h, half, sSb, sUb); break;
    default: scan_item<128, O_DT, kModeRun>(p, c, h, half, sSb, sUb); break;
  }
}

// ---- segment-parallel scan ----------------------------------------------------
// A batch of a few long sequences leaves most of the chip idle in the scan
// above: 16 heads x 8 slices of one sequence are 128 chains of 1,024 chunk
// steps each for 65,536 tokens.  The chunk step is affine in the state,
// S1 = M S0 + B with M = Diag(e^{G_C}) - Kbar^T W and B = Kbar^T Ut, so a
// sequence is cut into segments of kSegChunks chunks, run in three launches:
//  1. compose: every segment but the last runs its chain twice without
//     outputs, from S = I without Ut (giving its M) and from S = 0 (giving
//     its B), into `maps`;
//  2. prefix: per (sequence, head, 16 value columns), the states entering
//     segments 1.. in turn, S <- M S + B in fp32, into `sin`;
//  3. run: every segment runs its chain with outputs from its entering state
//     (the sequence's initial state for segment 0); the last one writes the
//     final state.
// Launches 1 and 3 are chains of kSegChunks steps over many more work-groups.
// Results differ from the single chain by rounding only (the bf16 operand
// rounding of the state inside each chain, and the fp32 products of step 2).
struct SegArgs {
  ScanArgs p;
  int n;                               // sequences (<= kSegSeqMax)
  int run0, run1, run2, run3, run4;    // first segment of sequence s (run4 = all segments)
  int cmp0, cmp1, cmp2, cmp3, cmp4;    // first composed segment of sequence s
  int splits;                          // work-groups per (segment, head) and 128 columns
  float *maps;                         // [segments][H][2][128][128] fp32: M, B
  float *sin;                          // [segments][H][128][128] fp32: state entering the segment
};

__device__ __forceinline__ int seq_of(int x, int a1, int a2, int a3, int n) {
  return (n > 1 && x >= a1) + (n > 2 && x >= a2) + (n > 3 && x >= a3);
}
__device__ __forceinline__ int pick(int s, int a0, int a1, int a2, int a3, int a4) {
  return s == 0 ? a0 : s == 1 ? a1 : s == 2 ? a2 : s == 3 ? a3 : a4;
}

// Work-group b -> (item, sub): the `subs` work-groups of one item share
// b mod 8, i.e. one XCD and its L2 (they read the same records).
__device__ __forceinline__ void seg_item(int b, int subs, int &item, int &sub) {
  const int group = b / (8 * subs);
  sub = (b / 8) % subs;
  item = group * 8 + (b % 8);
}

__global__ __launch_bounds__(kScanThreads) void kda_chunk_seg_compose_kernel(SegArgs a) {
  __shared__ __attribute__((aligned(16))) uint8_t sSb[4 * 8 * 64 * 16];
  __shared__ __attribute__((aligned(16))) uint8_t sUb[2 * 8 * 64 * 16];
  const ScanArgs &p = a.p;
  int item, sub;
  seg_item(blockIdx.x, 2 * a.splits, item, sub);
  const int h = item % p.num_heads;
  const int ci = item / p.num_heads;
  if (ci >= a.cmp4) return;
  const int s = seq_of(ci, a.cmp1, a.cmp2, a.cmp3, a.n);
  const int j = ci - pick(s, a.cmp0, a.cmp1, a.cmp2, a.cmp3, a.cmp4);
  const bool affine = sub >= a.splits;
  const int half = sub % a.splits;
  Chain c = sequence_chain(p, s, h);
  c.first += j * kSegChunks;
  c.tok_a += static_cast<int64_t>(j) * kSegChunks * kC;
  c.nchunks = static_cast<int>(imin64(imin64(kSegChunks, c.nchunks - j * kSegChunks), p.max_ch - c.first));
  c.init = nullptr;
  const int seg = pick(s, a.run0, a.run1, a.run2, a.run3, a.run4) + j;
  c.fin = a.maps + ((static_cast<size_t>(seg) * p.num_heads + h) * 2 + (affine ? 1 : 0)) * kD * kD;
  switch (a.splits) {
    case 8:
      if (affine) scan_item<16, SOPHIA_DTYPE_BF16, kModeComposeB>(p, c, h, half, sSb, sUb);
      else scan_item<16, SOPHIA_DTYPE_BF16, kModeComposeM>(p, c, h, half, sSb, sUb);
      break;
    case 4:
      if (affine) scan_item<32, SOPHIA_DTYPE_BF16, kModeComposeB>(p, c, h, half, sSb, sUb);
      else scan_item<32, SOPHIA_DTYPE_BF16, kModeComposeM>(p, c, h, half, sSb, sUb);
      break;
    case 2:
      if (affine) scan_item<64, SOPHIA_DTYPE_BF16, kModeComposeB>(p, c, h, half, sSb, sUb);
      else scan_item<64, SOPHIA_DTYPE_BF16, kModeComposeM>(p, c, h, half, sSb, sUb);
      break;
    default:
      if (affine) scan_item<128, SOPHIA_DTYPE_BF16, kModeComposeB>(p, c, h, half, sSb, sUb);
      else scan_item<128, SOPHIA_DTYPE_BF16, kModeComposeM>(p, c, h, half, sSb, sUb);
      break;
  }
}

// One 256-thread work-group per (sequence, head, 16 value columns).  A step
// S <- M S + B is 128 x 16 outputs on fp32 MFMA (16x16x4): wavefront w owns
// rows 32w .. 32w + 31 as two 16 x 16 tiles over 32 k-steps.  M is staged in
// LDS (rows padded to 132 floats: the 16 rows x 4 k of an A operand fall in
// distinct banks); the next step's M and B are loaded into registers while
// this step computes.
constexpr int kLdM = kD + 4;
__global__ __launch_bounds__(256) void kda_chunk_seg_prefix_kernel(SegArgs a) {
  __shared__ __attribute__((aligned(16))) float sM[kD * kLdM];
  __shared__ __attribute__((aligned(16))) float sS[2][kD][16];
  const ScanArgs &p = a.p;
  // The 8 slices of one (sequence, head) share blockIdx mod 8, i.e. one XCD,
  // whose L2 then serves each map to all of them.
  int sh, slice;
  seg_item(blockIdx.x, 8, sh, slice);
  const int h = sh % p.num_heads;
  const int s = sh / p.num_heads;
  if (s >= a.n) return;
  const int seg0 = pick(s, a.run0, a.run1, a.run2, a.run3, a.run4);
  const int nseg = pick(s + 1, a.run0, a.run1, a.run2, a.run3, a.run4) - seg0;
  if (nseg <= 1) return;
  const int t = threadIdx.x;
  const int w = t >> 6, l = t & 63, x = l & 15, y = l >> 4;
  const int col = 16 * slice + x;
  const Chain c = sequence_chain(p, s, h);
  {
    // the state entering segment 0: thread t copies row t / 2, 8 columns
    const int row = t >> 1, c8 = (t & 1) * 8;
    float *first_in = a.sin + (static_cast<size_t>(seg0) * p.num_heads + h) * kD * kD + row * kD + 16 * slice + c8;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float v = c.init ? c.init[row * kD + 16 * slice + c8 + i] : 0.f;
      sS[0][row][c8 + i] = v;
      first_in[i] = v;
    }
  }
  // M of segment `seg` into registers (piece i: row (t + 256 i) / 32, columns
  // 4 ((t + 256 i) % 32) .. +3) and the B values of this lane's C tiles.
  f4 mr[16];
  f4 br[2];
  const auto load_map = [&](size_t seg) {
    const float *M = a.maps + ((seg * p.num_heads + h) * 2) * kD * kD;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int idx = t + 256 * i;
      mr[i] = *reinterpret_cast<const f4 *>(M + (idx >> 5) * kD + 4 * (idx & 31));
    }
#pragma unroll
    for (int r = 0; r < 2; ++r)
#pragma unroll
      for (int i = 0; i < 4; ++i) br[r][i] = M[kD * kD + (32 * w + 16 * r + 4 * y + i) * kD + col];
  };
  load_map(static_cast<size_t>(seg0));
  int cur = 0;
  for (int j = 0; j + 1 < nseg; ++j) {
    const size_t seg = static_cast<size_t>(seg0 + j);
    __syncthreads();  // every wavefront is done with the previous M and S
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int idx = t + 256 * i;
      *reinterpret_cast<f4 *>(&sM[(idx >> 5) * kLdM + 4 * (idx & 31)]) = mr[i];
    }
    f4 acc[2] = {br[0], br[1]};
    __syncthreads();
    // the next map loads while this step computes
    if (j + 2 < nseg) load_map(seg + 1);
#pragma unroll 8
    for (int ks = 0; ks < kD / 4; ++ks) {
      const float b = sS[cur][4 * ks + y][x];
#pragma unroll
      for (int r = 0; r < 2; ++r) acc[r] = mfma_f32x4(sM[(32 * w + 16 * r + x) * kLdM + 4 * ks + y], b, acc[r]);
    }
    float *dst = a.sin + ((seg + 1) * p.num_heads + h) * kD * kD;
#pragma unroll
    for (int r = 0; r < 2; ++r)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = 32 * w + 16 * r + 4 * y + i;
        sS[cur ^ 1][row][x] = acc[r][i];
        dst[row * kD + col] = acc[r][i];
      }
    cur ^= 1;
  }
}

template <int O_DT>
__global__ __launch_bounds__(kScanThreads) void kda_chunk_seg_run_kernel(SegArgs a) {
  __shared__ __attribute__((aligned(16))) uint8_t sSb[4 * 8 * 64 * 16];
  __shared__ __attribute__((aligned(16))) uint8_t sUb[2 * 8 * 64 * 16];
  const ScanArgs &p = a.p;
  int item, half;
  seg_item(blockIdx.x, a.splits, item, half);
  const int h = item % p.num_heads;
  const int gi = item / p.num_heads;
  if (gi >= a.run4) return;
  const int s = seq_of(gi, a.run1, a.run2, a.run3, a.n);
  const int seg0 = pick(s, a.run0, a.run1, a.run2, a.run3, a.run4);
  const int nseg = pick(s + 1, a.run0, a.run1, a.run2, a.run3, a.run4) - seg0;
  const int j = gi - seg0;
  Chain c = sequence_chain(p, s, h);
  if (nseg > 1) {
    // A segmented sequence's segments all start from `sin` (segment 0's copy
    // of the initial state was made by the prefix launch, so a final state
    // that aliases the initial one is written only after it was read).
    c.first += j * kSegChunks;
    c.tok_a += static_cast<int64_t>(j) * kSegChunks * kC;
    c.nchunks = static_cast<int>(imin64(imin64(kSegChunks, c.nchunks - j * kSegChunks), p.max_ch - c.first));
    c.init = a.sin + (static_cast<size_t>(gi) * p.num_heads + h) * kD * kD;
    if (j + 1 < nseg) c.fin = nullptr;
  }
  switch (a.splits) {
    case 8: scan_item<16, O_DT, kModeRun>(p, c, h, half, sSb, sUb); break;
    case 4: scan_item<32, O_DT, kModeRun>(p, c, h, half, sSb, sUb); break;
    case 2: scan_item<64, O_DT, kModeRun>(p, c, h, half, sSb, sUb); break;
    default: scan_item<128, O_DT, kModeRun>(p, c, h, half, sSb, sUb); break;
  }
}

// ---- backward: forward states, reverse chunk scan, per-chunk gradients --------
// The chunk form of the backward (FlashKDA's chunk_kda_train_bwd, as
// FlashKDAFunction.backward calls it, ml/training/pretrain/engine/
// sm120_concurrent_ffn.py:301-373).  Per chunk, with S0 the state entering it
// and dS1 the gradient of the state leaving it:
//   dU  = A_qk^T dO + Kbar dS1
//   dS0 = Diag(e^Gamma) dS1 + Qg^T dO - W^T dU        (the reverse chunk scan)
// and once S0, U, dS1 and dU of every chunk are known, its gradients need
// nothing from the other chunks:
//   dQg = dO S0^T, dKbar = U dS1^T, dA_qk = tril(dO U^T), dXu = T^T dU,
//   dXw = T^T dW = -dXu S0^T (dW = -dU S0^T),
//   dA_kk = tril_strict(-T^T dT T^T) = tril_strict(-T^T tril_strict(dU U^T))
//   (dT = dW Xw^T + dU Xu^T = dU (T^-1 U)^T, Xw = beta Kg, Xu = beta V),
//   then back through A_kk = Diag(beta) P and A_qk with the sub-block
//   factors, and dg = the reverse cumulative sum of dG plus dGamma on every
//   row; the l2 norms', the gate's and the beta sigmoid's backward follow.
// Three kernels after the backward's instantiation of the intra kernel:
//  * kda_bwd_states_kernel: the forward scan keeping S0 and U of every chunk;
//  * kda_bwd_rscan_kernel: the reverse scan, same two roles as the forward
//    one: four wavefronts form dU (rows 16w..), four hold dS in fp32 MFMA
//    accumulators; it keeps dS1 and dU of every chunk and leaves dh0;
//  * kda_bwd_grad_kernel: one work-group of 512 threads per (chunk, head),
//    every product as a split bf16 product (about 16 mantissa bits, fp32
//    accumulation); it reads the raw q, k, g, beta and writes the final dq,
//    dk, dv, dg, dbeta.
struct BwdChunkArgs {
  ScanArgs p;                  // offsets, sizes, forward records, h0
  const uint8_t *brec;         // backward records
  const float *tpmat;          // [max_ch][H][64][64]: T lower, P^T strict upper
  float *s0, *u, *ds1, *du;    // [max_ch][H][128][128], [max_ch][H][64][128]
  const float *dht;            // [n_seqs][H][128][128] or NULL
  float *dh0;                  // [n_seqs][H][128][128] or NULL
  int splits;                  // work-groups (value-column slices) per (sequence, head): 2, 4 or 8
  const void *q, *k, *v;       // the forward's inputs (rows of v_stride elements of v_dtype)
  int64_t v_stride;
  int v_dtype;
  const void *g;
  int64_t g_stride;
  int g_dtype;
  const void *beta;
  int64_t beta_stride;
  int beta_dtype;
  const float *A_log, *dt_bias;
  float scale, lb;
  unsigned flags;
  const void *dout;
  int64_t do_stride;
  int do_dtype;
  void *dq, *dk;                      // gradients of q, k (element type grad_dtype)
  float *dg, *dbeta;                   // gradients of g, beta (fp32)
  void *dv;                            // gradient of v (element type grad_dtype)
  int grad_dtype;
};

// One (sequence, head, NVB value columns) of the forward scan that keeps S0
// and U of every chunk (the steps of scan_item without O, the records read at
// each chunk).
template <int NVB>
__device__ __forceinline__ void fstate_item(const BwdChunkArgs &a, const Chain &c, int h, int half, uint8_t *sSb,
                                            uint8_t *sUb) {
  constexpr int NT = NVB / 16;
  const ScanArgs &p = a.p;
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l = tid & 63, lr = l & 15, gq = l >> 4;
  const int nt0 = half * NT;
  const int nchunks = __builtin_amdgcn_readfirstlane(c.nchunks);
  const size_t H = static_cast<size_t>(p.num_heads);
  const size_t item0 = static_cast<size_t>(c.first) * H + h;
  if (wave < 4) {
    const int w = wave;
    for (int cc = 0; cc < nchunks; ++cc) {
      const size_t it = item0 + static_cast<size_t>(cc) * H;
      const uint8_t *rec = p.records + it * kRecBytes;
      u4 wn[4];
      u2 ut[NT];
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) wn[ks] = *reinterpret_cast<const u4 *>(rec + kOffW + ((w * 4 + ks) * 64 + l) * 16);
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) ut[nt] = *reinterpret_cast<const u2 *>(rec + kOffU + ((w * 8 + nt0 + nt) * 64 + l) * 8);
      float *uo = a.u + it * (kC * kD);
      lds_barrier();  // S of this chunk is published
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        f4 u = f4{__uint_as_float(ut[nt].x << 16), __uint_as_float(ut[nt].x & 0xffff0000u),
                  __uint_as_float(ut[nt].y << 16), __uint_as_float(ut[nt].y & 0xffff0000u)};
#pragma unroll
        for (int ks = 0; ks < 4; ++ks)
          u = mfma32(bits_to_bf8(wn[ks]), bits_to_bf8(*reinterpret_cast<const u4 *>(sSb + ((ks * NT + nt) * 64 + l) * 16)), u);
        *reinterpret_cast<u2 *>(sUb + (((w >> 1) * NT + nt) * 64 + l) * 16 + (w & 1) * 8) = pack4_bf16(u);
#pragma unroll
        for (int e = 0; e < 4; ++e) uo[(16 * w + 4 * gq + e) * kD + 16 * (nt0 + nt) + lr] = u[e];
      }
      lds_barrier();  // U is published
    }
    return;
  }
  const int sw = wave - 4;
  f4 S[2][NT];
#pragma unroll
  for (int mi = 0; mi < 2; ++mi)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
      for (int e = 0; e < 4; ++e)
        S[mi][nt][e] = c.init ? c.init[(32 * sw + 16 * mi + 4 * gq + e) * kD + 16 * (nt0 + nt) + lr] : 0.f;
  if (nchunks > 0) publish_state<NT>(S, sSb, sw, l);
  for (int cc = 0; cc < nchunks; ++cc) {
    const size_t it = item0 + static_cast<size_t>(cc) * H;
    const uint8_t *rec = p.records + it * kRecBytes;
    SFrags f;
    load_s(f, rec, sw, l, gq);
    float *so = a.s0 + it * (kD * kD);
#pragma unroll
    for (int mi = 0; mi < 2; ++mi)
#pragma unroll
      for (int nt = 0; nt < NT; ++nt)
#pragma unroll
        for (int e = 0; e < 4; ++e) so[(32 * sw + 16 * mi + 4 * gq + e) * kD + 16 * (nt0 + nt) + lr] = S[mi][nt][e];
    lds_barrier();  // S published (the U role forms U)
    state_update<NT>(f, S, sSb, sUb, sw, l);  // waits for U, updates S, publishes it
  }
}

// Sequence whose chains the work-groups of rank `rank` run in the backward's
// two scans: for a batch of at most kOrderMax sequences the longest first
// (most chunks; ties by index), so that the work-groups of a second round
// hold the short chains; `rank` itself for larger batches.  Lane i ranks
// sequence i against the others (one load per lane, a shuffle per sequence).
__device__ __forceinline__ int longest_first(const ScanArgs &p, int rank) {
  const int n = p.n_seqs;
  if (n > kOrderMax) return rank;
  const int lane = threadIdx.x & 63;
  int64_t ch = -1;
  if (lane < n) {
    const int64_t a0 = iclamp64(p.cu[lane], 0, p.total);
    const int64_t b0 = iclamp64(p.cu[lane + 1], a0, p.total);
    ch = (b0 - a0 + kC - 1) / kC;
  }
  const int c32 = static_cast<int>(ch);
  int r = 0;
  for (int j = 0; j < n; ++j) {
    const int cj = __shfl(c32, j, 64);
    r += (cj > c32 || (cj == c32 && j < lane)) ? 1 : 0;
  }
  const unsigned long long hit = __ballot(lane < n && r == rank);
  return hit ? __builtin_ctzll(hit) : rank;
}

__global__ __launch_bounds__(kScanThreads) void kda_bwd_states_kernel(BwdChunkArgs a) {
  __shared__ __attribute__((aligned(16))) uint8_t sSb[4 * 8 * 64 * 16];
  __shared__ __attribute__((aligned(16))) uint8_t sUb[2 * 8 * 64 * 16];
  const ScanArgs &p = a.p;
  if (p.total > 0)   // rows no sequence covers: zero gradients (no other kernel writes them)
    zero_rows_outside(p.cu, p.n_seqs, p.total, p.num_heads, a.dq, a.dk, a.dv, a.grad_dtype, a.dg, a.dbeta,
                      static_cast<int64_t>(blockIdx.x) * kScanThreads + threadIdx.x,
                      static_cast<int64_t>(gridDim.x) * kScanThreads);
  int item, half;
  seg_item(blockIdx.x, a.splits, item, half);
  const int h = item % p.num_heads;
  if (item / p.num_heads >= p.n_seqs) return;
  const int s = longest_first(p, item / p.num_heads);
  const Chain c = sequence_chain(p, s, h);
  switch (a.splits) {
    case 8: fstate_item<16>(a, c, h, half, sSb, sUb); break;
    case 4: fstate_item<32>(a, c, h, half, sSb, sUb); break;
    default: fstate_item<64>(a, c, h, half, sSb, sUb); break;
  }
}

// One (sequence, head, NVB value columns) of the reverse scan on 512 threads;
// the chunks of the sequence in reverse order.  Barriers pair as in
// scan_item: per chunk, dS published -> the dU role forms and publishes dU ->
// the state role updates dS and publishes it for the chunk before.
template <int NVB>
__device__ __forceinline__ void rscan_item(const BwdChunkArgs &a, const Chain &c, int s, int h, int half,
                                           uint8_t *sSb, uint8_t *sUb) {
  constexpr int NT = NVB / 16;
  const ScanArgs &p = a.p;
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l = tid & 63, lr = l & 15, gq = l >> 4;
  const int nt0 = half * NT;
  const int nchunks = __builtin_amdgcn_readfirstlane(c.nchunks);
  const size_t H = static_cast<size_t>(p.num_heads);
  const size_t item0 = static_cast<size_t>(c.first) * H + h;
  if (wave < 4) {
    const int w = wave;
    for (int cc = nchunks - 1; cc >= 0; --cc) {
      const size_t it = item0 + static_cast<size_t>(cc) * H;
      const uint8_t *br = a.brec + it * kBwdRecBytes;
      u4 at[2], kb[4], dob[2][NT];
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) at[ks] = *reinterpret_cast<const u4 *>(br + kBOffAt + ((w * 2 + ks) * 64 + l) * 16);
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) kb[ks] = *reinterpret_cast<const u4 *>(br + kBOffKbar + ((w * 4 + ks) * 64 + l) * 16);
#pragma unroll
      for (int ks = 0; ks < 2; ++ks)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
          dob[ks][nt] = *reinterpret_cast<const u4 *>(br + kBOffDo + ((ks * 8 + nt0 + nt) * 64 + l) * 16);
      float *duo = a.du + it * (kC * kD);
      lds_barrier();  // dS1 of this chunk is published
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        f4 d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) d = mfma32(bits_to_bf8(at[ks]), bits_to_bf8(dob[ks][nt]), d);
#pragma unroll
        for (int ks = 0; ks < 4; ++ks)
          d = mfma32(bits_to_bf8(kb[ks]), bits_to_bf8(*reinterpret_cast<const u4 *>(sSb + ((ks * NT + nt) * 64 + l) * 16)), d);
        *reinterpret_cast<u2 *>(sUb + (((w >> 1) * NT + nt) * 64 + l) * 16 + (w & 1) * 8) = pack4_bf16(d);
#pragma unroll
        for (int e = 0; e < 4; ++e) duo[(16 * w + 4 * gq + e) * kD + 16 * (nt0 + nt) + lr] = d[e];
      }
      lds_barrier();  // dU is published
    }
    return;
  }
  // state role: dS rows 32sw + 16mi + 4gq + e, column 16(nt0 + nt) + lr
  const int sw = wave - 4;
  const size_t sq = (static_cast<size_t>(s) * H + h) * kD * kD;
  f4 S[2][NT];
#pragma unroll
  for (int mi = 0; mi < 2; ++mi)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
      for (int e = 0; e < 4; ++e)
        S[mi][nt][e] = a.dht ? a.dht[sq + (32 * sw + 16 * mi + 4 * gq + e) * kD + 16 * (nt0 + nt) + lr] : 0.f;
  if (nchunks > 0) publish_state<NT>(S, sSb, sw, l);
  for (int cc = nchunks - 1; cc >= 0; --cc) {
    const size_t it = item0 + static_cast<size_t>(cc) * H;
    const uint8_t *br = a.brec + it * kBwdRecBytes;
    const float *gam = reinterpret_cast<const float *>(p.records + it * kRecBytes + kOffG);
    u4 qt[2][2], wt[2][2], dob[2][NT];
    f4 gm[2];
#pragma unroll
    for (int mi = 0; mi < 2; ++mi) {
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        qt[mi][ks] = *reinterpret_cast<const u4 *>(br + kBOffQt + (((2 * sw + mi) * 2 + ks) * 64 + l) * 16);
        wt[mi][ks] = *reinterpret_cast<const u4 *>(br + kBOffWt + (((2 * sw + mi) * 2 + ks) * 64 + l) * 16);
      }
      gm[mi] = *reinterpret_cast<const f4 *>(&gam[32 * sw + 16 * mi + 4 * gq]);
    }
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
#pragma unroll
      for (int nt = 0; nt < NT; ++nt)
        dob[ks][nt] = *reinterpret_cast<const u4 *>(br + kBOffDo + ((ks * 8 + nt0 + nt) * 64 + l) * 16);
    float *so = a.ds1 + it * (kD * kD);
#pragma unroll
    for (int mi = 0; mi < 2; ++mi)
#pragma unroll
      for (int nt = 0; nt < NT; ++nt)
#pragma unroll
        for (int e = 0; e < 4; ++e) so[(32 * sw + 16 * mi + 4 * gq + e) * kD + 16 * (nt0 + nt) + lr] = S[mi][nt][e];
    lds_barrier();  // dS1 published (the dU role forms dU)
    lds_barrier();  // dU published
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      bf8 ub[2];
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) ub[ks] = bits_to_bf8(*reinterpret_cast<const u4 *>(sUb + ((ks * NT + nt) * 64 + l) * 16));
#pragma unroll
      for (int mi = 0; mi < 2; ++mi) {
        f4 v = S[mi][nt] * gm[mi];
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) v = mfma32(bits_to_bf8(qt[mi][ks]), bits_to_bf8(dob[ks][nt]), v);
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) v = mfma32(bits_to_bf8(wt[mi][ks]), ub[ks], v);
        S[mi][nt] = v;
      }
    }
    publish_state<NT>(S, sSb, sw, l);
  }
  if (a.dh0) {
#pragma unroll
    for (int mi = 0; mi < 2; ++mi)
#pragma unroll
      for (int nt = 0; nt < NT; ++nt)
#pragma unroll
        for (int e = 0; e < 4; ++e)
          a.dh0[sq + (32 * sw + 16 * mi + 4 * gq + e) * kD + 16 * (nt0 + nt) + lr] = S[mi][nt][e];
  }
}

__global__ __launch_bounds__(kScanThreads) void kda_bwd_rscan_kernel(BwdChunkArgs a) {
  __shared__ __attribute__((aligned(16))) uint8_t sSb[4 * 8 * 64 * 16];
  __shared__ __attribute__((aligned(16))) uint8_t sUb[2 * 8 * 64 * 16];
  const ScanArgs &p = a.p;
  int item, half;
  seg_item(blockIdx.x, a.splits, item, half);
  const int h = item % p.num_heads;
  if (item / p.num_heads >= p.n_seqs) return;
  const int s = longest_first(p, item / p.num_heads);
  const Chain c = sequence_chain(p, s, h);
  switch (a.splits) {
    case 8: rscan_item<16>(a, c, s, h, half, sSb, sUb); break;
    case 4: rscan_item<32>(a, c, s, h, half, sSb, sUb); break;
    default: rscan_item<64>(a, c, s, h, half, sSb, sUb); break;
  }
}

// Products of the gradient kernel.  Plain bf16 operands here leave dg, and
// the per-head sums dA_log / ddt_bias over it, 10-40x further from the
// float64 reference (dg is a reverse cumulative sum of terms that cancel).
// Split products: x = hi + lo with hi = bf16(x) and lo = bf16(x - hi) keeps
// ~16 mantissa bits, and hi.hi + hi.lo + lo.hi (lo.lo, below 2^-16 of the
// product, dropped) on bf16 MFMAs with fp32 accumulation takes three 16x16x32
// MFMAs where fp32 operands take eight 16x16x4 ones (step i of lane group g
// covering k = 8g + i).  Lane group g holds k = 8g .. 8g + 7 of a 16x16x32
// operand, so the same eight values per lane form the fragment in either.
struct Sp8 {
  bf8 hi, lo;
};
__device__ __forceinline__ Sp8 split8(const float (&x)[8]) {
  Sp8 s;
  s.hi = pack8(x);
  float r[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) r[i] = x[i] - static_cast<float>(s.hi[i]);
  s.lo = pack8(r);
  return s;
}
__device__ __forceinline__ f4 mma3(const Sp8 &x, const Sp8 &y, f4 acc) {
  acc = mfma32(x.lo, y.hi, acc);
  acc = mfma32(x.hi, y.lo, acc);
  return mfma32(x.hi, y.hi, acc);
}

// The same split for 4 values, as bf16 bits: hi and lo words of two pairs.
__device__ __forceinline__ void split4(const f4 &x, u2 &hi, u2 &lo) {
  float r[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) r[i] = x[i] - static_cast<float>(static_cast<__bf16>(x[i]));
  hi = u2{pack_bf16x2(x[0], x[1]), pack_bf16x2(x[2], x[3])};
  lo = u2{pack_bf16x2(r[0], r[1]), pack_bf16x2(r[2], r[3])};
}

__device__ __forceinline__ void load8f(const float *src, float (&x)[8]) {
  const f4 a = *reinterpret_cast<const f4 *>(src), b = *reinterpret_cast<const f4 *>(src + 4);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    x[i] = a[i];
    x[4 + i] = b[i];
  }
}

constexpr int kLdG = 132;   // fp32 row strides of the gradient kernel's LDS tiles
constexpr int kLdS = 68;
constexpr int kLdQ = 20;    // q^ column block: rows 4 apart land 16 banks apart
constexpr int kGradThreads = 512;
constexpr size_t kGradLdsFloats =
    3 * 64 * kLdG + 2 * 64 * kLdS + 2 * 16 * kLdG + 64 * kLdQ + 64 + 128 + 4 * 128 + 2 * 64 + 4 * 64;

// One (chunk, head) of the per-chunk gradients on 512 threads: wavefronts w
// and w + 4 (one pair per SIMD) share the chunk rows 16w .. 16w + 15 of every
// product whose rows are chunk rows.
//
// Since U = T (Xu - Xw S0), the gradient of T, dT = dW Xw^T + dU Xu^T with
// dW = -dU S0^T, equals dU (T^{-1} U)^T, so that
//   dA_kk = tril_strict(-T^T dT T^T) = tril_strict(-T^T tril_strict(dU U^T)),
//   dXw = T^T dW = -dXu S0^T with dXu = T^T dU:
// neither dW nor dT is formed.
//
// LDS holds G, k^ and dU (then dXu, then phase II's exchange) as [64][128]
// tiles and two [64][64] tiles that each keep a lower-triangular matrix in
// place and a strictly lower one transposed into the upper triangle: T with
// P (later dP), and dA_qk with dU U^T.  Step 2 gives the pair the key blocks
// of dA_qk and dU U^T by parity; step 3 the column blocks of dXu.  Phase II
// walks the 16-channel column blocks with the pair in two roles: the state
// wavefront (u = 0) forms dQg = dO S0^T and dXw = -dXu S0^T of block i from
// one pass over 16 rows of S0, while the chunk wavefront (u = 1) forms
// dKbar = U dS1^T and the products through A_qk and P of block i and
// finishes block i - 1 (dq^, dk^, dG into G's dead columns) from the state
// wavefront's results.  The state matrices stream through a [32][128] block
// prefetched into registers one block ahead; every tile issues the loads of
// all its K-steps before its first product.
// GD: element type of dq, dk and dv.
template <int GD>
__global__ __launch_bounds__(kGradThreads) void kda_bwd_grad_kernel(BwdChunkArgs a) {
  extern __shared__ __attribute__((aligned(16))) float gsm[];
  float *sG = gsm;                  // [64][kLdG] G (natural log); dG column blocks as phase II ends them
  float *sKh = sG + 64 * kLdG;      // [64][kLdG] k^
  float *sDX = sKh + 64 * kLdG;     // [64][kLdG] dU, then dXu; phase II [2][4][64][8] exchange
  float *sTP = sDX + 64 * kLdG;     // [64][kLdS] T[r][j] (j <= r) at [r][j]; P / dP [r][j] (j < r) at [j][r]
  float *sAT = sTP + 64 * kLdS;     // [64][kLdS] dA_qk (j <= r) at [r][j]; (dU U^T)[r][j] (j < r) at [j][r]
  float *sSl = sAT + 64 * kLdS;     // [32][kLdG] rows 16i .. of S0 (0..15) and dS1 (16..31), split (see slb)
  float *sQb = sSl + 2 * 16 * kLdG; // [64][kLdQ] q^ columns 16i .. 16i + 15
  float *sBt = sQb + 64 * kLdQ;     // [64] beta
  float *sDg0 = sBt + 64;           // [128] e^Gamma sum_v dS1 S0
  float *sDgW = sDg0 + 128;         // [4][128] per-row-block sums of dKbar Kbar
  float *sDb = sDgW + 4 * 128;      // [2][64] dbeta of each wavefront of a pair
  float *sRq = sDb + 2 * 64;        // [64] q^ = q sRq (scale / |q| with the l2 norm)
  float *sRk = sRq + 64;            // [64] k^ = k sRk
  float *sIq = sRk + 64;            // [64] 1 / |q|^2 where the l2 norm's backward has the rank-1 term, else 0
  float *sIk = sIq + 64;            // [64] the same flag for k (1 or 0)
  // dq^ sRq of every row (phase II): rows 0..31 in the dA_qk tile (read
  // into registers by then), rows 32..63 behind the exchange
  const auto dQrow = [&](int r) { return r < 32 ? sAT + r * kLdG : sDX + 4096 + (r - 32) * kLdG; };
  const ScanArgs &p = a.p;
  const int H = p.num_heads;
  const int h = static_cast<int>(blockIdx.x % static_cast<unsigned>(H));
  const int cidx = static_cast<int>(blockIdx.x / static_cast<unsigned>(H));
  if (cidx >= p.max_ch) return;
  int s, first;
  chunk_of(p.cu, p.n_seqs, p.total, cidx, s, first);
  if (s >= p.n_seqs) return;
  const int64_t seq_a = iclamp64(p.cu[s], 0, p.total);
  const int64_t seq_b = iclamp64(p.cu[s + 1], seq_a, p.total);
  const int64_t tok0 = seq_a + static_cast<int64_t>(cidx - first) * kC;
  const int len = static_cast<int>(imin64(kC, seq_b - tok0));
  const size_t it = static_cast<size_t>(cidx) * H + h;
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int w = wave & 3, u = wave >> 2;
  const int l = tid & 63, lr = l & 15, gq = l >> 4;
  const int rb = 16 * w;
  const int st0 = w >> 1;   // T^T[m][k] = T[k][m] vanishes for k < m: row blocks 2, 3 skip K-step 0
  const auto tok_off = [&](int r) { return (tok0 + r) * static_cast<int64_t>(H) + h; };
  const int64_t vrow = static_cast<int64_t>(h) * kD;
  const float *S0 = a.s0 + it * (kD * kD);
  const float *dS1 = a.ds1 + it * (kD * kD);
  const float *Um = a.u + it * (kC * kD);
  const float *dUm = a.du + it * (kC * kD);
  const f4 z4 = {0.f, 0.f, 0.f, 0.f};
  const auto Gat = [&](int r, int c) { return sG[r * kLdG + c]; };
  const auto Kat = [&](int r, int c) { return sKh[r * kLdG + c]; };
  // Thread tid's share of a 32-row block of a [.][128] matrix: rows (tid >> 5)
  // and (tid >> 5) + 16, columns 4 (tid & 31) .. + 3.
  const int blk_r = tid >> 5, blk_c = 4 * (tid & 31);

  // ---- 1. the log-decay (the gate applied), k^ (the norms of q and k) and
  //         dU rows (zero past len), T and P, beta; the dO rows of this row
  //         block; the U rows of the first key block
  const bool l2 = (a.flags & SOPHIA_KDA_QK_L2NORM) != 0;
  const bool gate = (a.flags & SOPHIA_KDA_GATE_IN_KERNEL) != 0;
  const float ea = gate ? __expf(a.A_log[h]) : 0.f;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int r = blk_r + 16 * q;
    f4 gv = z4, kv = z4, qv = z4, dv = z4;
    if (r < len) {
      const int64_t ro = (tok0 + r) * a.v_stride + vrow + blk_c;
      qv = load4(a.q, ro, a.v_dtype);
      kv = load4(a.k, ro, a.v_dtype);
      gv = load4(a.g, (tok0 + r) * a.g_stride + vrow + blk_c, a.g_dtype);
      if (gate) {
#pragma unroll
        for (int e = 0; e < 4; ++e) gv[e] = kda_log_decay(gv[e], ea, a.dt_bias[h * kD + blk_c + e], a.lb);
      }
      dv = *reinterpret_cast<const f4 *>(&dUm[r * kD + blk_c]);
    }
    float sq = qv[0] * qv[0] + qv[1] * qv[1] + qv[2] * qv[2] + qv[3] * qv[3];
    float sk = kv[0] * kv[0] + kv[1] * kv[1] + kv[2] * kv[2] + kv[3] * kv[3];
#pragma unroll
    for (int off = 1; off < 32; off <<= 1) {   // the 32 threads of row r
      sq += __shfl_xor(sq, off, 64);
      sk += __shfl_xor(sk, off, 64);
    }
    const float lq = sqrtf(sq), lk = sqrtf(sk);
    const float rk = l2 ? 1.f / fmaxf(lk, 1e-12f) : 1.f;
    if ((tid & 31) == 0) {
      sRq[r] = l2 ? a.scale / fmaxf(lq, 1e-12f) : a.scale;
      sRk[r] = rk;
      sIq[r] = l2 && lq >= 1e-12f ? 1.f / (lq * lq) : 0.f;
      sIk[r] = l2 && lk >= 1e-12f ? 1.f : 0.f;
    }
    *reinterpret_cast<f4 *>(&sG[r * kLdG + blk_c]) = gv;
    *reinterpret_cast<f4 *>(&sKh[r * kLdG + blk_c]) = kv * rk;
    *reinterpret_cast<f4 *>(&sDX[r * kLdG + blk_c]) = dv;
  }
  {
    const float *tp = a.tpmat + it * (kC * kC);   // already in sTP's layout
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int i = tid + kGradThreads * q, r = i >> 4, c = 4 * (i & 15);
      *reinterpret_cast<f4 *>(&sTP[r * kLdS + c]) = *reinterpret_cast<const f4 *>(&tp[4 * i]);
    }
  }
  if (tid < kC) {
    float b = 0.f;
    if (tid < len) {
      b = load_elem(a.beta, (tok0 + tid) * a.beta_stride + h, a.beta_dtype);
      if (a.flags & SOPHIA_KDA_BETA_SIGMOID) b = sigmoid_f(b);
    }
    sBt[tid] = b;
  }
  float xo[4][8];
  {
    const int r = rb + lr;
    const int64_t oo = (tok0 + r) * a.do_stride + vrow;
#pragma unroll
    for (int st = 0; st < 4; ++st) {
      const int kb = 32 * st + 8 * gq;
      if (r < len) {
        const f4 u0 = load4(a.dout, oo + kb, a.do_dtype), u1 = load4(a.dout, oo + kb + 4, a.do_dtype);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          xo[st][i] = u0[i];
          xo[st][4 + i] = u1[i];
        }
      } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) xo[st][i] = 0.f;
      }
    }
  }
  Sp8 xos[4];   // the dO rows, split (see mma3)
#pragma unroll
  for (int st = 0; st < 4; ++st) xos[st] = split8(xo[st]);
  // U rows of key block ib (rows past len are finite and meet zero dO / dU rows)
  float un[4][8];
  const auto fetch_keys = [&](int ib) {
#pragma unroll
    for (int st = 0; st < 4; ++st) load8f(Um + (16 * ib + lr) * kD + 32 * st + 8 * gq, un[st]);
  };
  if (u <= w) fetch_keys(u);
  // v at the positions of this wavefront's dXu tiles (rows 16w + 4gq + e, columns 16 (u + 2k) + lr)
  float vown[4][4];
#pragma unroll
  for (int k = 0; k < 4; ++k)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int r = rb + 4 * gq + e;
      vown[k][e] = r < len ? load_elem(a.v, (tok0 + r) * a.v_stride + vrow + 16 * (u + 2 * k) + lr, a.v_dtype) : 0.f;
    }
  lds_barrier();
  // G = cumulative log-decay: each quarter of the threads scans 16 rows of a
  // channel, then the rows of a quarter add the totals of the quarters before.
  {
    const int c = tid & 127, qr = tid >> 7;
    float acc = 0.f;
#pragma unroll 8
    for (int r = 16 * qr; r < 16 * qr + 16; ++r) {
      acc += sG[r * kLdG + c];
      sG[r * kLdG + c] = acc;
    }
    lds_barrier();
    float base = 0.f;
    for (int q = 0; q < qr; ++q) base += sG[(16 * q + 15) * kLdG + c];
    lds_barrier();
    if (qr > 0) {
#pragma unroll 8
      for (int r = 16 * qr; r < 16 * qr + 16; ++r) sG[r * kLdG + c] += base;
    }
  }

  // ---- 2. per key block ib <= w with ib = u (mod 2): dA_qk = tril(dO U^T)
  //         and the strictly lower part of dU U^T
  {
    Sp8 xds[4];   // dU rows of this row block, split
#pragma unroll
    for (int st = 0; st < 4; ++st) {
      float xd[8];
      load8f(sDX + (rb + lr) * kLdG + 32 * st + 8 * gq, xd);
      xds[st] = split8(xd);
    }
#pragma unroll
    for (int k2 = 0; k2 < 2; ++k2) {
      const int ib = u + 2 * k2;
      if (ib > w) continue;
      f4 aq = z4, ay = z4;
#pragma unroll
      for (int st = 0; st < 4; ++st) {
        const Sp8 us = split8(un[st]);
        aq = mma3(xos[st], us, aq);
        ay = mma3(xds[st], us, ay);
      }
      if (k2 == 0 && ib + 2 <= w) fetch_keys(ib + 2);
      const int j = 16 * ib + lr;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int r = rb + 4 * gq + e;
        if (j <= r) sAT[r * kLdS + j] = aq[e];
        if (j < r) sAT[j * kLdS + r] = ay[e];
      }
    }
  }
  // The blocks of phase II's step i (i = -1 .. 7): rows 16 (i + 1) .. of S0
  // for the state wavefronts, rows 16 i .. of dS1 and q^'s columns 16 i ..
  // for the chunk wavefronts.
  f4 pre[2], qpre = z4;
  const int q_r = tid >> 2, q_c = 4 * (tid & 3);
  const auto fetch2 = [&](int i) {
    if (i < 7) {
      pre[0] = *reinterpret_cast<const f4 *>(S0 + (16 * (i + 1) + blk_r) * kD + blk_c);
      pre[1] = *reinterpret_cast<const f4 *>(dS1 + (16 * (i + 1) + blk_r) * kD + blk_c);
    }
    if (i >= 0 && tid < 256 && q_r < len)
      qpre = load4(a.q, (tok0 + q_r) * a.v_stride + vrow + 16 * i + q_c, a.v_dtype);
  };
  fetch2(-1);

  // ---- 3. dXu = T^T dU (rows of this row block, column blocks u + 2k); dv;
  //         beta's term sum_v dXu v
  float ta[2][8];   // T^T rows of this row block
#pragma unroll
  for (int st = 0; st < 2; ++st) {
    const int kb = 32 * st + 8 * gq, m = rb + lr;
#pragma unroll
    for (int i = 0; i < 8; ++i) ta[st][i] = m <= kb + i ? sTP[(kb + i) * kLdS + m] : 0.f;
  }
  Sp8 tas[2];
#pragma unroll
  for (int st = 0; st < 2; ++st) tas[st] = split8(ta[st]);
  float dbr[4] = {0.f, 0.f, 0.f, 0.f};
  f4 dxu[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int c = 16 * (u + 2 * k) + lr;
    dxu[k] = z4;
#pragma unroll
    for (int st = 0; st < 2; ++st) {
      if (st < st0) continue;
      const int kb = 32 * st + 8 * gq;
      float y[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) y[i] = sDX[(kb + i) * kLdG + c];
      dxu[k] = mma3(tas[st], split8(y), dxu[k]);
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int r = rb + 4 * gq + e;
      const float bt = sBt[r];
      dbr[e] += dxu[k][e] * vown[k][e];
      if (r < len) store_elem(a.dv, tok_off(r) * kD + c, GD, bt * dxu[k][e]);
    }
  }
  lds_barrier();   // dU is read; dA_qk and dU U^T are complete
#pragma unroll
  for (int k = 0; k < 4; ++k)
#pragma unroll
    for (int e = 0; e < 4; ++e) sDX[(rb + 4 * gq + e) * kLdG + 16 * (u + 2 * k) + lr] = dxu[k][e];

  // ---- 4. dA_kk = tril_strict(-T^T Y), Y = tril_strict(dU U^T), for key
  //         blocks ib = u (mod 2); beta's term sum_j dA_kk P; dP = beta dA_kk
#pragma unroll
  for (int k2 = 0; k2 < 2; ++k2) {
    const int ib = u + 2 * k2;
    if (ib > w) continue;
    // B[k][n] = Y[k][16 ib + n] (16 ib + n < k) at [16 ib + n][k]
    const int n = 16 * ib + lr;
    f4 acc = z4;
#pragma unroll
    for (int st = 0; st < 2; ++st) {
      if (st < st0) continue;
      const int kb = 32 * st + 8 * gq;
      float y[8];
      load8f(sAT + n * kLdS + kb, y);
#pragma unroll
      for (int i = 0; i < 8; ++i)
        if (kb + i <= n) y[i] = 0.f;
      acc = mma3(tas[st], split8(y), acc);
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int r = rb + 4 * gq + e;
      if (n < r) {
        const float dA = -acc[e];
        dbr[e] += dA * sTP[n * kLdS + r];
        sTP[n * kLdS + r] = sBt[r] * dA;
      }
    }
  }
  lds_barrier();   // dXu and dP are complete

  // ---- 5. (phase II) column blocks: in step i the state wavefronts form
  //         the state products of block i + 1 (dQg e^G, dXw, dKbar) and the
  //         chunk wavefronts the products through A_qk and P of block i,
  //         finishing it from the state wavefronts' results of step i - 1.  For rows r of
  //         block w the products through A_qk and P split e^{G_r - G_j} =
  //         e^{G_r - ref_w} e^{ref_w - G_j} (the first <= 1, the second <= 1
  //         for j before block w and <= e^80 inside it), and so do key rows j
  //         of block w with r >= 16w.  Keys j < 16 (w + 1) take the K-steps
  //         below kq, queries r >= 16 w those from st0.
  // The S0 and dS1 rows of a block are split once, as they are stashed: row
  // r of sSl holds the 128 hi bf16 of the row, then its 128 lo bf16 (split8's
  // split), so every wavefront reads MFMA operands with no conversion.  The
  // stash also forms dGamma's state term e^{Gamma_c} sum_v S0[c][v] dS1[c][v]
  // for the channels c of the block it stashes.
  uint8_t *const slb = reinterpret_cast<uint8_t *>(sSl);
  const auto sl_put = [&](int row, const f4 &x) {
    u2 hi, lo;
    split4(x, hi, lo);
    *reinterpret_cast<u2 *>(slb + row * (kLdG * 4) + 2 * blk_c) = hi;
    *reinterpret_cast<u2 *>(slb + row * (kLdG * 4) + 256 + 2 * blk_c) = lo;
  };
  const auto sl_get = [&](int row, int col) {
    Sp8 x;
    x.hi = bits_to_bf8(*reinterpret_cast<const u4 *>(slb + row * (kLdG * 4) + 2 * col));
    x.lo = bits_to_bf8(*reinterpret_cast<const u4 *>(slb + row * (kLdG * 4) + 256 + 2 * col));
    return x;
  };
  const auto stash2 = [&](int i) {
    if (i < 7) {   // S0 and dS1 of block i + 1
      sl_put(blk_r, pre[0]);
      sl_put(16 + blk_r, pre[1]);
      float d = ((pre[0][0] * pre[1][0]) + (pre[0][1] * pre[1][1])) + ((pre[0][2] * pre[1][2]) + (pre[0][3] * pre[1][3]));
#pragma unroll
      for (int off = 1; off < 32; off <<= 1) d += __shfl_xor(d, off, 64);   // the 32 threads of row blk_r
      if ((tid & 31) == 0) {
        const int c = 16 * (i + 1) + blk_r;
        sDg0[c] = d * __expf(Gat(kC - 1, c));
      }
    }
    if (i >= 0 && tid < 256) {   // q^ of block i
      const float rq = sRq[q_r];
#pragma unroll
      for (int e = 0; e < 4; ++e) sQb[q_r * kLdQ + q_c + e] = qpre[e] * rq;
    }
  };
  // dKbar of a block, from the state wavefronts to the chunk wavefronts: T / P
  // tile, unused in phase II (the chunk wavefronts keep dP in registers).
  float *sX2 = sTP;
  float *sX = sDX;
  if (u == 0) {
    // state wavefronts: dXu and U rows of this row block
    Sp8 xdus[4], xus[4];
#pragma unroll
    for (int st = 0; st < 4; ++st) {
      float xdu[8], xu[8];
      load8f(sDX + (rb + lr) * kLdG + 32 * st + 8 * gq, xdu);
      xdus[st] = split8(xdu);
      if (rb + lr < len) {
        load8f(Um + (rb + lr) * kD + 32 * st + 8 * gq, xu);
      } else {
#pragma unroll
        for (int k = 0; k < 8; ++k) xu[k] = 0.f;
      }
      xus[st] = split8(xu);
    }
    lds_barrier();   // dXu is read: its tile takes the exchange
    for (int i = -1; i < 8; ++i) {
      stash2(i);
      if (i < 7) fetch2(i + 1);
      lds_barrier();
      if (i < 7) {
        const int nb = i + 1, c = 16 * nb + lr;
        f4 dq = z4, dxw = z4;
#pragma unroll
        for (int st = 0; st < 4; ++st) {
          const Sp8 ss = sl_get(lr, 32 * st + 8 * gq);
          dq = mma3(xos[st], ss, dq);
          dxw = mma3(xdus[st], ss, dxw);
        }
        f4 xq, xw;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          xq[e] = dq[e] * __expf(Gat(rb + 4 * gq + e, c));   // through Qg = q^ e^G
          xw[e] = -dxw[e];
        }
        float *x = sX + (((nb & 1) * 4 + w) * 64 + l) * 8;
        *reinterpret_cast<f4 *>(x) = xq;
        *reinterpret_cast<f4 *>(x + 4) = xw;
        f4 dkb = z4;   // dKbar = U dS1^T: rows of this row block, channels c
#pragma unroll
        for (int st = 0; st < 4; ++st) dkb = mma3(xus[st], sl_get(16 + lr, 32 * st + 8 * gq), dkb);
        *reinterpret_cast<f4 *>(sX2 + (((nb & 1) * 4 + w) * 64 + l) * 4) = dkb;
      }
      lds_barrier();   // the blocks and the exchange are read
    }
  } else {
    // chunk wavefronts: dA_qk and dP rows / columns of this row block.  The
    // products over chunk rows k take K-step st's slot e of a lane at row
    // kperm(st, e): rows 4 apart in the lane groups, so that the per-lane
    // reads of G and k^ rows below land 16 banks apart (the same rows in
    // both operands, so the products are unchanged).
    const auto kperm = [&](int st, int e) { return 32 * st + 16 * (e >> 2) + 4 * gq + (e & 3); };
    const int m = rb + lr;
    Sp8 xas[2], xats[2], xps[2], xpts[2];
#pragma unroll
    for (int st = 0; st < 2; ++st) {
      float xa[8], xat[8], xp[8], xpt[8];
#pragma unroll
      for (int h2 = 0; h2 < 2; ++h2) {
        const f4 a4 = *reinterpret_cast<const f4 *>(sAT + m * kLdS + kperm(st, 4 * h2));
        const f4 p4 = *reinterpret_cast<const f4 *>(sTP + m * kLdS + kperm(st, 4 * h2));
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          xa[4 * h2 + e] = a4[e];
          xpt[4 * h2 + e] = p4[e];
        }
      }
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const int kk = kperm(st, k);
        if (kk > m) xa[k] = 0.f;                               // dA_qk[m][k], k <= m
        xat[k] = kk >= m ? sAT[kk * kLdS + m] : 0.f;          // dA_qk[k][m]
        if (kk <= m) xpt[k] = 0.f;                             // dP[k][m] (k > m)
        xp[k] = kk < m ? sTP[kk * kLdS + m] : 0.f;            // dP[m][k] (k < m)
      }
      // the same in every column block
      xas[st] = split8(xa);
      xats[st] = split8(xat);
      xps[st] = split8(xp);
      xpts[st] = split8(xpt);
    }
    lds_barrier();   // matches the state wavefronts' barrier
    // The column-block loop with the row block a compile-time constant W, so
    // that which K-steps a wavefront takes and the masks it needs are known
    // to the compiler (no branches inside the loop).
    const auto chunk_loop = [&](auto wc) {
      constexpr int W = decltype(wc)::value;
      constexpr int RB = 16 * W, JMAX = 16 * (W + 1), KQ = W < 2 ? 1 : 2, ST0 = W >> 1;
      // dG and dk^ of the previous block, written over G's and k^'s columns
      // once every wavefront has read them (after the next barrier)
      float pg[4] = {0.f, 0.f, 0.f, 0.f}, pk[4] = {0.f, 0.f, 0.f, 0.f};
      for (int i = -1; i < 8; ++i) {
        if (i >= 1) {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int r = RB + 4 * gq + e, c = 16 * (i - 1) + lr;
            sG[r * kLdG + c] = pg[e];
            sKh[r * kLdG + c] = pk[e];
          }
        }
        stash2(i);
        if (i < 7) fetch2(i + 1);
        lds_barrier();
        if (i >= 0) {
          const int c = 16 * i + lr;
          const float rwc = W == 0 ? 0.f : Gat(RB - 1, c);
          const float gam = Gat(kC - 1, c);
          f4 c1 = z4, c2 = z4, c34 = z4;
#pragma unroll
          for (int st = 0; st < 2; ++st) {
            if (st < KQ) {
              float y[8];
#pragma unroll
              for (int k = 0; k < 8; ++k) {
                const int j = kperm(st, k);
                y[k] = j < JMAX ? Kat(j, c) * __expf(rwc - Gat(j, c)) : 0.f;
              }
              const Sp8 ys = split8(y);
              c1 = mma3(xas[st], ys, c1);
              c2 = mma3(xps[st], ys, c2);
            }
            if (st >= ST0) {
              float yq[8], yk[8];
#pragma unroll
              for (int k = 0; k < 8; ++k) {
                const int r = kperm(st, k);
                const float f = r >= RB ? __expf(Gat(r, c) - rwc) : 0.f;
                yq[k] = sQb[r * kLdQ + lr] * f;
                yk[k] = Kat(r, c) * f;
              }
              c34 = mma3(xats[st], split8(yq), c34);
              c34 = mma3(xpts[st], split8(yk), c34);
            }
          }
          // finish block i with the state wavefronts' dQg e^G, dXw and dKbar
          const float *x = sX + (((i & 1) * 4 + W) * 64 + l) * 8;
          const f4 xq = *reinterpret_cast<const f4 *>(x), xw = *reinterpret_cast<const f4 *>(x + 4);
          const f4 dkb = *reinterpret_cast<const f4 *>(sX2 + (((i & 1) * 4 + W) * 64 + l) * 4);
          float part = 0.f;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int r = RB + 4 * gq + e;
            const float g = Gat(r, c);
            const float eg = __expf(g), f = __expf(gam - g), af = __expf(g - rwc), bq = __expf(rwc - g);
            const float kv = Kat(r, c), qv = sQb[r * kLdQ + lr], bt = sBt[r];
            const float dkbar = dkb[e] * f;                   // through Kbar = k^ e^{Gamma - G}
            const float dkg = bt * xw[e] * eg + af * c2[e];   // through Kg = k^ e^G
            const float dkr = bq * c34[e];                    // through the k^ e^{-G} factor
            const float dqv = xq[e] + af * c1[e];
            part += dkbar * kv;
            dbr[e] += xw[e] * kv * eg;
            pg[e] = qv * dqv + kv * (dkg - dkbar - dkr);      // dG
            pk[e] = dkbar + dkg + dkr;                        // dk^
            dQrow(r)[c] = dqv * sRq[r];
          }
          part += lane_xor16(part);
          part += lane_xor32(part);
          if (gq == 0) sDgW[W * kD + c] = part;
        }
        lds_barrier();   // the blocks, the exchange and G's and k^'s columns 16 i .. are read
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int r = RB + 4 * gq + e, c = 16 * 7 + lr;
        sG[r * kLdG + c] = pg[e];
        sKh[r * kLdG + c] = pk[e];
      }
    };
    switch (w) {
      case 0: chunk_loop(std::integral_constant<int, 0>{}); break;
      case 1: chunk_loop(std::integral_constant<int, 1>{}); break;
      case 2: chunk_loop(std::integral_constant<int, 2>{}); break;
      default: chunk_loop(std::integral_constant<int, 3>{}); break;
    }
  }
  // The output pass's q, k and gate-input rows, issued here so that their
  // latency overlaps the last barrier and the suffix sums below.
  f4 zv[4], qv[4], kv[4], gbias = z4;
  if (gate) gbias = *reinterpret_cast<const f4 *>(&a.dt_bias[h * kD + blk_c]);
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int r = blk_r + 16 * q;
    zv[q] = qv[q] = kv[q] = z4;
    if (r < len) {
      const int64_t ro = (tok0 + r) * a.v_stride + vrow + blk_c;
      qv[q] = load4(a.q, ro, a.v_dtype);
      kv[q] = load4(a.k, ro, a.v_dtype);
      if (gate) zv[q] = load4(a.g, (tok0 + r) * a.g_stride + vrow + blk_c, a.g_dtype);
    }
  }
  lds_barrier();   // dG and dk^ are complete

  // ---- 6. dbeta; dg = reverse cumulative sum of dG + dGamma
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    float x = dbr[e];
#pragma unroll
    for (int off = 1; off < 16; off <<= 1) x += __shfl_xor(x, off, 64);
    if (lr == 0) sDb[u * 64 + rb + 4 * gq + e] = x;
  }
  // Suffix sums within each quarter of the rows (16 rows, a channel per
  // thread); the rows of a quarter then add the totals of the quarters after it.
  {
    const int c = tid & 127, r0 = (tid >> 7) * 16;
    float acc = 0.f;
#pragma unroll 8
    for (int r = r0 + 15; r >= r0; --r) {
      acc += sG[r * kLdG + c];
      sG[r * kLdG + c] = acc;
    }
  }
  lds_barrier();
  if (tid >= 256 && tid < 256 + kC) {
    const int r = tid - 256;
    if (r < len) {
      float db = sDb[r] + sDb[64 + r];
      if (a.flags & SOPHIA_KDA_BETA_SIGMOID) db *= sBt[r] * (1.f - sBt[r]);
      a.dbeta[tok_off(r)] = db;
    }
  }
  // dg, dq and dk rows.  dg of the log-decay is the suffix sum plus dGamma;
  // through the gate g = lb sigmoid(e^A_log (z + dt_bias)), dz = dg lb s (1 - s) e^A_log.
  // The l2 norms' backward: dq = dq^ sRq - q (q^ . dq^) / |q|^2 and
  // dk = (dk^ - k^ (k^ . dk^)) / |k| = dk^ sRk - k sRk^2 (k^ . dk^), with
  // q^ . dq^ = q . (dq^ sRq) and k^ . dk^ = sRk (k . dk^): sums over the 32
  // threads of a row.
  {
    f4 dgam, tail[4];
    tail[3] = z4;
#pragma unroll
    for (int q = 2; q >= 0; --q) tail[q] = tail[q + 1] + *reinterpret_cast<const f4 *>(&sG[16 * (q + 1) * kLdG + blk_c]);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int cc = blk_c + e;
      dgam[e] = sDg0[cc] + ((sDgW[cc] + sDgW[kD + cc]) + (sDgW[2 * kD + cc] + sDgW[3 * kD + cc]));
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int r = blk_r + 16 * q;
      const f4 dqs = *reinterpret_cast<const f4 *>(dQrow(r) + blk_c);
      const f4 dks = *reinterpret_cast<const f4 *>(&sKh[r * kLdG + blk_c]);
      float sq = qv[q][0] * dqs[0] + qv[q][1] * dqs[1] + qv[q][2] * dqs[2] + qv[q][3] * dqs[3];
      float sk = kv[q][0] * dks[0] + kv[q][1] * dks[1] + kv[q][2] * dks[2] + kv[q][3] * dks[3];
#pragma unroll
      for (int off = 1; off < 32; off <<= 1) {
        sq += __shfl_xor(sq, off, 64);
        sk += __shfl_xor(sk, off, 64);
      }
      if (r >= len) continue;
      const float rk = sRk[r];
      f4 d = *reinterpret_cast<const f4 *>(&sG[r * kLdG + blk_c]) + dgam + tail[q];
      if (gate) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float sg = sigmoid_f(ea * (zv[q][e] + gbias[e]));
          d[e] *= a.lb * sg * (1.f - sg) * ea;
        }
      }
      const int64_t o = tok_off(r) * kD + blk_c;
      *reinterpret_cast<f4 *>(&a.dg[o]) = d;
      store4(a.dq, o, GD, dqs - qv[q] * (sIq[r] * sq));
      store4(a.dk, o, GD, dks * rk - kv[q] * (sIk[r] * rk * rk * rk * sk));
    }
  }
}

inline size_t seg_bytes(int64_t total_tokens, int num_heads) {
  return static_cast<size_t>(max_segments(total_tokens)) * num_heads * 3 * kD * kD * sizeof(float);
}

// Dynamic LDS above the default limit is enabled once per (kernel, device),
// under a lock: launches may come from several host threads and devices.
constexpr int kMaxDevices = 64;
// Sets a kernel's dynamic LDS limit once per device (KEY names the kernel).
template <class KEY>
int ensure_lds(const void *fn, size_t bytes) {
  static std::mutex mu;
  static bool done[kMaxDevices] = {};
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess)
    return set_error(SOPHIA_ERR_HIP, "kda_chunk: hipGetDevice: %s", hipGetErrorString(e));
  std::lock_guard<std::mutex> lock(mu);
  if (dev >= 0 && dev < kMaxDevices && done[dev]) return SOPHIA_OK;
  e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(bytes));
  if (e != hipSuccess)
    return set_error(SOPHIA_ERR_HIP, "kda_chunk: cannot set LDS size: %s", hipGetErrorString(e));
  if (dev >= 0 && dev < kMaxDevices) done[dev] = true;
  return SOPHIA_OK;
}
template <int QKV_DT, int G_DT, bool GATE, bool BWD>
struct IntraKey {};
template <int GD>
struct GradKey {};

template <int QKV_DT, int G_DT, bool GATE>
int ensure_intra_lds() {
  return ensure_lds<IntraKey<QKV_DT, G_DT, GATE, false>>(
      reinterpret_cast<const void *>(&kda_chunk_intra_kernel<QKV_DT, G_DT, GATE>), kSmIntra);
}

template <int QKV_DT, int G_DT, bool GATE>
int launch_intra(dim3 grid, hipStream_t st, const IntraArgs &ia) {
  if (const int rc = ensure_intra_lds<QKV_DT, G_DT, GATE>()) return rc;
  hipLaunchKernelGGL((kda_chunk_intra_kernel<QKV_DT, G_DT, GATE>), grid, dim3(kThreads), kSmIntra, st, ia);
  return check_launch("kda_chunk_intra");
}

template <int G_DT, bool GATE>
struct ConvIntraKey {};

template <int G_DT, bool GATE>
int launch_conv_intra(dim3 grid, hipStream_t st, const IntraArgs &ia) {
  if (const int rc = ensure_lds<ConvIntraKey<G_DT, GATE>>(
          reinterpret_cast<const void *>(&kda_chunk_conv_intra_kernel<G_DT, GATE>), kSmIntra))
    return rc;
  hipLaunchKernelGGL((kda_chunk_conv_intra_kernel<G_DT, GATE>), grid, dim3(kThreads), kSmIntra, st, ia);
  return check_launch("kda_chunk_conv_intra");
}

template <int QKV_DT, int G_DT, bool GATE>
int launch_intra_bwd(dim3 grid, hipStream_t st, const IntraArgs &ia) {
  if (const int rc = ensure_lds<IntraKey<QKV_DT, G_DT, GATE, true>>(
          reinterpret_cast<const void *>(&kda_chunk_intra_bwd_kernel<QKV_DT, G_DT, GATE>), kSmIntraBwd))
    return rc;
  hipLaunchKernelGGL((kda_chunk_intra_bwd_kernel<QKV_DT, G_DT, GATE>), grid, dim3(kThreads), kSmIntraBwd, st, ia);
  return check_launch("kda_chunk_intra_bwd");
}

template <int O_DT>
void launch_scan(dim3 grid, hipStream_t st, const ScanArgs &sa) {
  hipLaunchKernelGGL((kda_chunk_scan_kernel<O_DT>), grid, dim3(kScanThreads), 0, st, sa);
}

inline size_t align256(size_t b) { return (b + 255) & ~static_cast<size_t>(255); }

}  // namespace

// Scratch of the chunk-form backward, per (chunk, head): the forward and the
// backward record, the T / P tile, S0 and dS1, U and dU.
size_t chunk_bwd_scratch_bytes(int64_t total_tokens, int n_seqs, int num_heads) {
  const size_t items = static_cast<size_t>(max_chunks(total_tokens, n_seqs)) * num_heads;
  return align256(kTrashBytes) + align256(items * kRecBytes) + align256(items * kBwdRecBytes) +
         align256(items * kC * kC * 4) + 2 * align256(items * kD * kD * 4) + 2 * align256(items * kC * kD * 4);
}

int chunk_bwd_run(const ChunkBwdIO &io, void *scratch, hipStream_t st) {
  const int H = io.num_heads;
  const int64_t max_ch = max_chunks(io.total, io.n_seqs);
  if (max_ch <= 0) return SOPHIA_OK;
  SOPHIA_REQUIRE(max_ch * H <= 0x7fffffff, "kda_chunk_bwd: grid too large");
  const size_t items = static_cast<size_t>(max_ch) * H;
  uint8_t *w = static_cast<uint8_t *>(scratch);
  const auto carve = [&w](size_t bytes) {
    uint8_t *p = w;
    w += align256(bytes);
    return p;
  };
  void *trash = carve(kTrashBytes);
  uint8_t *records = carve(items * kRecBytes);
  uint8_t *brec = carve(items * kBwdRecBytes);
  float *tpmat = reinterpret_cast<float *>(carve(items * kC * kC * 4));
  float *s0 = reinterpret_cast<float *>(carve(items * kD * kD * 4));
  float *ds1 = reinterpret_cast<float *>(carve(items * kD * kD * 4));
  float *u = reinterpret_cast<float *>(carve(items * kC * kD * 4));
  float *du = reinterpret_cast<float *>(carve(items * kC * kD * 4));

  // 1. records (forward and backward), T and P
  if (io.total > 0) {
    const auto a16 = [](const void *ptr) { return reinterpret_cast<uintptr_t>(ptr) % 16 == 0; };
    const int lines = io.qkv_dtype == SOPHIA_DTYPE_BF16 && io.qkv_stride % 8 == 0 && a16(io.q) && a16(io.k) &&
                      a16(io.v);
    IntraArgs ia{io.q, io.k, io.v, io.qkv_stride, io.qkv_dtype, io.g, io.g_stride, io.g_dtype, io.beta,
                 io.beta_stride, io.beta_dtype, io.A_log, io.dt_bias, io.scale, io.lb, io.flags,
                 io.cu, io.n_seqs, io.total, H, max_ch, records, lines,
                 brec, tpmat, io.dout, io.do_stride, io.do_dtype};
    const dim3 grid(static_cast<unsigned>(items));
    const bool gate = (io.flags & SOPHIA_KDA_GATE_IN_KERNEL) != 0;
    const int key = (io.qkv_dtype == SOPHIA_DTYPE_BF16) * 4 + (io.g_dtype == SOPHIA_DTYPE_BF16) * 2 + gate;
    constexpr int F = SOPHIA_DTYPE_F32, B = SOPHIA_DTYPE_BF16;
    int rc = SOPHIA_OK;
    switch (key) {
      case 0: rc = launch_intra_bwd<F, F, false>(grid, st, ia); break;
      case 1: rc = launch_intra_bwd<F, F, true>(grid, st, ia); break;
      case 2: rc = launch_intra_bwd<F, B, false>(grid, st, ia); break;
      case 3: rc = launch_intra_bwd<F, B, true>(grid, st, ia); break;
      case 4: rc = launch_intra_bwd<B, F, false>(grid, st, ia); break;
      case 5: rc = launch_intra_bwd<B, F, true>(grid, st, ia); break;
      case 6: rc = launch_intra_bwd<B, B, false>(grid, st, ia); break;
      default: rc = launch_intra_bwd<B, B, true>(grid, st, ia); break;
    }
    if (rc) return rc;
  }
  // 2-3. forward states and the reverse scan: `splits` slices of the value
  // columns per (sequence, head), as many as keep every work-group resident.
  int device = 0, cus = 256;
  if (hipGetDevice(&device) == hipSuccess)
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess) cus = 256;
  const int64_t pairs = static_cast<int64_t>(io.n_seqs) * H;
  // (at least 2: a 128-column slice does not fit these kernels' registers).
  // With the chains taken longest first (at most kOrderMax sequences) two
  // rounds of work-groups pay: thinner slices store less per chunk step, and
  // the second round holds the short chains (benchmark batch: 2 slices
  // 258.7 + 147.3 us, 4 slices 156.1 + 107.1 us, 8 slices 205.7 + 142.5 us).
  int splits = 2;
  const int64_t room = io.n_seqs <= kOrderMax ? 2 * static_cast<int64_t>(cus) : cus;
  while (splits < 8 && pairs * splits * 2 <= room) splits *= 2;
  const int64_t sblocks = (pairs + 7) / 8 * 8 * splits;
  SOPHIA_REQUIRE(sblocks <= 0x7fffffff, "kda_chunk_bwd: grid too large");
  BwdChunkArgs a{};
  a.p = ScanArgs{io.cu, io.n_seqs, io.total, H, max_ch, records, io.h0, nullptr, io.n_seqs, nullptr, nullptr, 0,
                 trash, 0xfedcba9876543210ull, 1, 0, 0, 0, 0, 0, 0, 0, 0, 0, 1, 1, 1, 1};
  a.brec = brec; a.tpmat = tpmat;
  a.s0 = s0; a.u = u; a.ds1 = ds1; a.du = du;
  a.dht = io.dht; a.dh0 = io.dh0; a.splits = splits;
  a.q = io.q; a.k = io.k; a.v = io.v; a.v_stride = io.qkv_stride; a.v_dtype = io.qkv_dtype;
  a.g = io.g; a.g_stride = io.g_stride; a.g_dtype = io.g_dtype;
  a.beta = io.beta; a.beta_stride = io.beta_stride; a.beta_dtype = io.beta_dtype;
  a.A_log = io.A_log; a.dt_bias = io.dt_bias; a.scale = io.scale; a.lb = io.lb; a.flags = io.flags;
  a.dout = io.dout; a.do_stride = io.do_stride; a.do_dtype = io.do_dtype;
  a.dq = io.dq; a.dk = io.dk; a.dg = io.dg; a.dbeta = io.dbeta; a.dv = io.dv; a.grad_dtype = io.grad_dtype;
  hipLaunchKernelGGL(kda_bwd_states_kernel, dim3(static_cast<unsigned>(sblocks)), dim3(kScanThreads), 0, st, a);
  if (const int rc = check_launch("kda_bwd_states")) return rc;
  hipLaunchKernelGGL(kda_bwd_rscan_kernel, dim3(static_cast<unsigned>(sblocks)), dim3(kScanThreads), 0, st, a);
  if (const int rc = check_launch("kda_bwd_rscan")) return rc;
  // 4. per-chunk gradients
  if (io.total == 0) return SOPHIA_OK;
  const size_t glds = kGradLdsFloats * sizeof(float);
  const auto grad = [&](auto gd) {
    constexpr int GD = decltype(gd)::value;
    if (const int rc = ensure_lds<GradKey<GD>>(reinterpret_cast<const void *>(&kda_bwd_grad_kernel<GD>), glds))
      return rc;
    hipLaunchKernelGGL(kda_bwd_grad_kernel<GD>, dim3(static_cast<unsigned>(items)), dim3(kGradThreads), glds, st, a);
    return check_launch("kda_bwd_grad");
  };
  return io.grad_dtype == SOPHIA_DTYPE_BF16 ? grad(std::integral_constant<int, SOPHIA_DTYPE_BF16>{})
                                            : grad(std::integral_constant<int, SOPHIA_DTYPE_F32>{});
}

}  // namespace sophia

using namespace sophia;

extern "C" size_t sophia_kda_chunk_workspace_size(int64_t total_tokens, int n_seqs, int num_heads,
                                                  int head_dim) {
  if (total_tokens < 0 || n_seqs <= 0 || num_heads <= 0 || head_dim != kD) return 0;
  return kTrashBytes +
         static_cast<size_t>(max_chunks(total_tokens, n_seqs)) * num_heads * kRecBytes +
         seg_bytes(total_tokens, num_heads);
}

namespace {
// The ShortConv fused into the prefill (sophia_kda_conv_chunk_fwd).
struct ConvIO {
  const float *weight;  // [3 H 128][4] fp32
  float *state;         // [n_state_slots][3 H 128][3] fp32, or NULL
  int read_history;
};

// The body of the prefill entry points: `workspace` is either the caller's
// buffer or this library's static scratch (sophia_kda_chunk_fwd_no_alloc);
// with `conv`, q, k, v are the rows before the fused ShortConv.
int chunk_fwd_impl(const void *q, const void *k, const void *v, int64_t qkv_row_stride, int qkv_dtype,
                   const void *g, int64_t g_row_stride, int g_dtype, const void *beta,
                   int64_t beta_row_stride, int beta_dtype, const float *A_log, const float *dt_bias,
                   float scale, float lower_bound, unsigned flags, const int32_t *cu_seqlens,
                   const int32_t *cu_seqlens_host, int n_seqs, int64_t total_tokens, int num_heads,
                   int head_dim, const float *initial_state, float *final_state, int n_state_slots,
                   const int32_t *state_slots, void *o, int64_t o_row_stride, void *workspace,
                   size_t workspace_bytes, void *stream, const ConvIO *conv = nullptr) {
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
  SOPHIA_REQUIRE(qkv_row_stride % 4 == 0 && g_row_stride % 4 == 0 && o_row_stride % 4 == 0,
                 "kda_chunk_fwd: q/k/v/g/o row strides must be multiples of 4 elements");
  SOPHIA_REQUIRE(total_tokens == 0 ||
                     (reinterpret_cast<uintptr_t>(o) % (qkv_dtype == SOPHIA_DTYPE_BF16 ? 8 : 16)) == 0,
                 "kda_chunk_fwd: o must be aligned to 4 elements");
  SOPHIA_REQUIRE(((uintptr_t)workspace % 256) == 0, "kda_chunk_fwd: workspace must be 256-byte aligned");
  SOPHIA_REQUIRE(n_state_slots >= 0, "kda_chunk_fwd: n_state_slots must be >= 0");
  if (cu_seqlens_host) {
    bool ok = cu_seqlens_host[0] >= 0 && cu_seqlens_host[n_seqs] <= total_tokens;
    for (int i = 0; ok && i < n_seqs; ++i) ok = cu_seqlens_host[i] <= cu_seqlens_host[i + 1];
    SOPHIA_REQUIRE(ok, "kda_chunk_fwd: cu_seqlens_host is not a non-decreasing offset array in [0, total]");
  }
  const size_t need = sophia_kda_chunk_workspace_size(total_tokens, n_seqs, num_heads, head_dim);
  if (workspace_bytes < need)
    return set_error(SOPHIA_ERR_WORKSPACE, "kda_chunk_fwd: workspace %zu bytes < required %zu",
                     workspace_bytes, need);
  const int64_t max_ch = max_chunks(total_tokens, n_seqs);
  SOPHIA_REQUIRE(max_ch <= 0x7fffffff, "kda_chunk_fwd: too many chunks");
  hipStream_t st = static_cast<hipStream_t>(stream);
  uint8_t *trash = static_cast<uint8_t *>(workspace);
  uint8_t *records = trash + kTrashBytes;
  int rc = SOPHIA_OK;
  const auto a16 = [](const void *ptr) { return reinterpret_cast<uintptr_t>(ptr) % 16 == 0; };
  const int lines = qkv_dtype == SOPHIA_DTYPE_BF16 && qkv_row_stride % 8 == 0 && a16(q) && a16(k) && a16(v);
  IntraArgs ia{q, k, v, qkv_row_stride, qkv_dtype, g, g_row_stride, g_dtype, beta,
               beta_row_stride, beta_dtype, A_log, dt_bias, scale, lower_bound, flags,
               cu_seqlens, n_seqs, total_tokens, num_heads, max_ch, records, lines};
  if (conv) {
    SOPHIA_REQUIRE(lines || total_tokens == 0,
                   "kda_conv_chunk_fwd: x must be bf16 rows, 16-byte aligned, row stride a multiple of 8");
    ia.conv_w = conv->weight;
    ia.conv_state = conv->state;
    ia.conv_slots = state_slots;
    ia.conv_n_slots = conv->state ? n_state_slots : 0;
    ia.conv_read = conv->read_history;
  }

  if (max_ch > 0 && total_tokens > 0) {
    SOPHIA_REQUIRE(max_ch * num_heads <= 0x7fffffff, "kda_chunk_fwd: grid too large");
    const dim3 grid(static_cast<unsigned>(max_ch * num_heads));
    const bool gate = (flags & SOPHIA_KDA_GATE_IN_KERNEL) != 0;
    const int key = (qkv_dtype == SOPHIA_DTYPE_BF16) * 4 + (g_dtype == SOPHIA_DTYPE_BF16) * 2 + gate;
    constexpr int F = SOPHIA_DTYPE_F32, B = SOPHIA_DTYPE_BF16;
    switch (conv ? 8 + (g_dtype == SOPHIA_DTYPE_BF16) * 2 + gate : key) {
      case 8: rc = launch_conv_intra<F, false>(grid, st, ia); break;
      case 9: rc = launch_conv_intra<F, true>(grid, st, ia); break;
      case 10: rc = launch_conv_intra<B, false>(grid, st, ia); break;
      case 11: rc = launch_conv_intra<B, true>(grid, st, ia); break;
      case 0: rc = launch_intra<F, F, false>(grid, st, ia); break;
      case 1: rc = launch_intra<F, F, true>(grid, st, ia); break;
      case 2: rc = launch_intra<F, B, false>(grid, st, ia); break;
      case 3: rc = launch_intra<F, B, true>(grid, st, ia); break;
      case 4: rc = launch_intra<B, F, false>(grid, st, ia); break;
      case 5: rc = launch_intra<B, F, true>(grid, st, ia); break;
      case 6: rc = launch_intra<B, B, false>(grid, st, ia); break;
      default: rc = launch_intra<B, B, true>(grid, st, ia); break;
    }
    if (rc) return rc;
  }
  if (conv && conv->state) {
    // after the intra kernel has read the old histories
    const int threads = 3 * num_heads * (kD / 8);
    hipLaunchKernelGGL(kda_conv_history_kernel, dim3(static_cast<unsigned>((threads + 255) / 256),
                                                     static_cast<unsigned>(n_seqs)), dim3(256), 0, st, ia);
    if (const int rc2 = check_launch("kda_conv_history")) return rc2;
  }
  // The state scan is sequential over the chunks of a sequence: the 128
  // value columns of each (sequence, head) are split over 1, 2, 4 or 8
  // work-groups (plan_scan), so that a small batch still spreads its
  // critical path over the chip.  The host copy of the offsets shapes this
  // plan; results do not depend on it, except that a few long sequences are
  // cut into segments (plan_segments; rounding differences only, and
  // SOPHIA_KDA_SCAN_NO_SEGMENTS keeps one chain per sequence).
  int device = 0, cus = 256;
  if (hipGetDevice(&device) == hipSuccess)
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess) cus = 256;
  const SegPlan sp = plan_segments(cu_seqlens_host, n_seqs, num_heads, cus, total_tokens, flags);
  if (sp.on) {
    float *maps = reinterpret_cast<float *>(records + static_cast<size_t>(max_ch) * num_heads * kRecBytes);
    float *sin = maps + static_cast<size_t>(max_segments(total_tokens)) * num_heads * 2 * kD * kD;
    SegArgs a{{cu_seqlens, n_seqs, total_tokens, num_heads, max_ch, records, initial_state, final_state,
               n_state_slots, state_slots, o, o_row_stride, trash, 0, 1, 0, 0, 0, 0, 0, 0, 0, 0, 0, 1, 1, 1, 1},
              n_seqs,
              sp.run[0], sp.run[1], sp.run[2], sp.run[3], sp.run[4],
              sp.cmp[0], sp.cmp[1], sp.cmp[2], sp.cmp[3], sp.cmp[4],
              sp.cmp_splits, maps, sin};
    const int64_t cmp_blocks = (static_cast<int64_t>(sp.cmp[n_seqs]) * num_heads + 7) / 8 * 8 * 2 * sp.cmp_splits;
    if (cmp_blocks > 0) {
      hipLaunchKernelGGL(kda_chunk_seg_compose_kernel, dim3(static_cast<unsigned>(cmp_blocks)),
                         dim3(kScanThreads), 0, st, a);
      if (const int rc2 = check_launch("kda_chunk_seg_compose")) return rc2;
      hipLaunchKernelGGL(kda_chunk_seg_prefix_kernel, dim3(static_cast<unsigned>((n_seqs * num_heads + 7) / 8 * 64)),
                         dim3(256), 0, st, a);
      if (const int rc2 = check_launch("kda_chunk_seg_prefix")) return rc2;
    }
    a.splits = sp.run_splits;
    const int64_t run_blocks = (static_cast<int64_t>(sp.run[n_seqs]) * num_heads + 7) / 8 * 8 * sp.run_splits;
    if (qkv_dtype == SOPHIA_DTYPE_BF16)
      hipLaunchKernelGGL(kda_chunk_seg_run_kernel<SOPHIA_DTYPE_BF16>, dim3(static_cast<unsigned>(run_blocks)),
                         dim3(kScanThreads), 0, st, a);
    else
      hipLaunchKernelGGL(kda_chunk_seg_run_kernel<SOPHIA_DTYPE_F32>, dim3(static_cast<unsigned>(run_blocks)),
                         dim3(kScanThreads), 0, st, a);
    return check_launch("kda_chunk_seg_run");
  }
  const ScanPlan pl = plan_scan(cu_seqlens_host, n_seqs, num_heads, cus, total_tokens);
  SOPHIA_REQUIRE(pl.blocks > 0 && pl.blocks <= 0x7fffffff, "kda_chunk_fwd: grid too large");
  ScanArgs sa{cu_seqlens, n_seqs, total_tokens, num_heads, max_ch, records,
              initial_state, final_state, n_state_slots, state_slots, o, o_row_stride, trash,
              pl.order_bits, pl.n_cls,
              pl.block[0], pl.block[1], pl.block[2], pl.block[3],
              pl.rank[0], pl.rank[1], pl.rank[2], pl.rank[3], pl.rank[4],
              pl.splits[0], pl.splits[1], pl.splits[2], pl.splits[3]};
  const dim3 sgrid(static_cast<unsigned>(pl.blocks));
  if (qkv_dtype == SOPHIA_DTYPE_BF16)
    launch_scan<SOPHIA_DTYPE_BF16>(sgrid, st, sa);
  else
    launch_scan<SOPHIA_DTYPE_F32>(sgrid, st, sa);
  return check_launch("kda_chunk_scan");
}

// ---- static scratch for callers that cannot allocate -------------------------
// One array per device (each device that loads this library holds its own
// copy until the process ends).  Host code never passes `scratch` itself to a
// kernel: its host-side name is not a device address.  The device address is
// looked up once per device with hipGetSymbolAddress and kept in
// g_scratch_ptr.  Nothing in it needs to start at zero: the intra kernel
// writes every record before the scan reads it, and the scratch rows are
// only written.
constexpr size_t kStaticScratchBytes = SOPHIA_KDA_CHUNK_NO_ALLOC_MAX_BYTES;
__device__ __align__(256) uint8_t scratch[kStaticScratchBytes];

std::mutex g_scratch_mu;
void *g_scratch_ptr[kMaxDevices] = {};

int static_scratch(void **out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess)
    return set_error(SOPHIA_ERR_HIP, "kda_chunk_fwd_no_alloc: hipGetDevice: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices)
    return set_error(SOPHIA_ERR_INVALID, "kda_chunk_fwd_no_alloc: device %d beyond %d", dev, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void *ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr)
      return set_error(SOPHIA_ERR_HIP, "kda_chunk_fwd_no_alloc: hipGetSymbolAddress(scratch) failed: %s",
                       hipGetErrorString(e));
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return SOPHIA_OK;
}
}  // namespace

extern "C" int sophia_kda_chunk_fwd(const void *q, const void *k, const void *v,
                                    int64_t qkv_row_stride, int qkv_dtype, const void *g,
                                    int64_t g_row_stride, int g_dtype, const void *beta,
                                    int64_t beta_row_stride, int beta_dtype, const float *A_log,
                                    const float *dt_bias, float scale, float lower_bound,
                                    unsigned flags, const int32_t *cu_seqlens,
                                    const int32_t *cu_seqlens_host, int n_seqs,
                                    int64_t total_tokens, int num_heads, int head_dim,
                                    const float *initial_state, float *final_state,
                                    int n_state_slots, const int32_t *state_slots, void *o,
                                    int64_t o_row_stride,
                                    void *workspace, size_t workspace_bytes, void *stream) {
  return chunk_fwd_impl(q, k, v, qkv_row_stride, qkv_dtype, g, g_row_stride, g_dtype, beta,
                        beta_row_stride, beta_dtype, A_log, dt_bias, scale, lower_bound, flags,
                        cu_seqlens, cu_seqlens_host, n_seqs, total_tokens, num_heads, head_dim,
                        initial_state, final_state, n_state_slots, state_slots, o, o_row_stride,
                        workspace, workspace_bytes, stream);
}

extern "C" int sophia_kda_conv_chunk_fwd(const void *x_q, const void *x_k, const void *x_v,
                                         int64_t x_row_stride, int qkv_dtype, const float *conv_weight,
                                         float *conv_state, int kernel_size, int read_history, const void *g,
                                         int64_t g_row_stride, int g_dtype, const void *beta,
                                         int64_t beta_row_stride, int beta_dtype, const float *A_log,
                                         const float *dt_bias, float scale, float lower_bound, unsigned flags,
                                         const int32_t *cu_seqlens, const int32_t *cu_seqlens_host, int n_seqs,
                                         int64_t total_tokens, int num_heads, int head_dim,
                                         const float *initial_state, float *final_state, int n_state_slots,
                                         const int32_t *state_slots, void *o, int64_t o_row_stride,
                                         void *workspace, size_t workspace_bytes, void *stream) {
  const auto a16 = [](const void *ptr) { return reinterpret_cast<uintptr_t>(ptr) % 16 == 0; };
  SOPHIA_REQUIRE(kernel_size == 4, "kda_conv_chunk_fwd: kernel_size must be 4 (got %d)", kernel_size);
  SOPHIA_REQUIRE(qkv_dtype == SOPHIA_DTYPE_BF16, "kda_conv_chunk_fwd: x must be bf16");
  SOPHIA_REQUIRE(conv_weight && a16(conv_weight), "kda_conv_chunk_fwd: conv_weight must be 16-byte aligned");
  SOPHIA_REQUIRE(!conv_state || a16(conv_state), "kda_conv_chunk_fwd: conv_state must be 16-byte aligned");
  SOPHIA_REQUIRE(n_seqs > 0 && n_seqs <= 65535, "kda_conv_chunk_fwd: n_seqs must be in [1, 65535]");
  const ConvIO conv{conv_weight, conv_state, read_history != 0};
  return chunk_fwd_impl(x_q, x_k, x_v, x_row_stride, qkv_dtype, g, g_row_stride, g_dtype, beta,
                        beta_row_stride, beta_dtype, A_log, dt_bias, scale, lower_bound, flags,
                        cu_seqlens, cu_seqlens_host, n_seqs, total_tokens, num_heads, head_dim,
                        initial_state, final_state, n_state_slots, state_slots, o, o_row_stride,
                        workspace, workspace_bytes, stream, &conv);
}

extern "C" int sophia_kda_chunk_fwd_no_alloc(const void *q, const void *k, const void *v,
                                             int64_t qkv_row_stride, int qkv_dtype, const void *g,
                                             int64_t g_row_stride, int g_dtype, const void *beta,
                                             int64_t beta_row_stride, int beta_dtype,
                                             const float *A_log, const float *dt_bias, float scale,
                                             float lower_bound, unsigned flags,
                                             const int32_t *cu_seqlens,
                                             const int32_t *cu_seqlens_host, int n_seqs,
                                             int64_t total_tokens, int num_heads, int head_dim,
                                             const float *initial_state, float *final_state,
                                             int n_state_slots, const int32_t *state_slots, void *o,
                                             int64_t o_row_stride, void *stream) {
  const size_t need = sophia_kda_chunk_workspace_size(total_tokens, n_seqs, num_heads, head_dim);
  SOPHIA_REQUIRE(need > 0, "kda_chunk_fwd_no_alloc: bad total_tokens / n_seqs / num_heads / head_dim");
  if (need > kStaticScratchBytes)
    return set_error(SOPHIA_ERR_WORKSPACE,
                     "kda_chunk_fwd_no_alloc: this batch needs %zu bytes of scratch, more than the "
                     "%zu-byte static buffer (use sophia_kda_chunk_fwd with a workspace)",
                     need, kStaticScratchBytes);
  void *ws = nullptr;
  if (const int rc = static_scratch(&ws)) return rc;
  return chunk_fwd_impl(q, k, v, qkv_row_stride, qkv_dtype, g, g_row_stride, g_dtype, beta,
                        beta_row_stride, beta_dtype, A_log, dt_bias, scale, lower_bound, flags,
                        cu_seqlens, cu_seqlens_host, n_seqs, total_tokens, num_heads, head_dim,
                        initial_state, final_state, n_state_slots, state_slots, o, o_row_stride, ws,
                        kStaticScratchBytes, stream);
}
