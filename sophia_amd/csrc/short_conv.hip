// ShortConv: depthwise causal conv1d (kernel K <= 4) + SiLU with a rolling
// fp32 history cache, over a packed ragged batch.
//
// Semantics follow CausalDepthwiseConv1d.forward (ml/runtime/model/attention.py:32-60):
//   seq = cat(history[c, 0:K-1], x[:, c]);  y[t, c] = silu(sum_j w[c, j] * seq[t + j]);
//   next_history = seq[-(K-1):].
// One launch covers every channel of the fused q|k|v projection output
// (3 x 2048 channels at Sophia's shape), which is how SophiaKDA._short_convolution
// (attention.py:226-258) applies three convs and writes conv_state[:, 0..2].
//
// Memory-bound: each thread owns 8 consecutive channels (16 B of bf16) and
// walks 16 consecutive packed rows, keeping the K-1 previous samples in
// registers, so every x element is read from HBM once and y written once.
#include "common.hpp"

namespace sophia {
namespace {

constexpr int kVec = 8;        // channels per thread
constexpr int kVecsPerBlock = 64;
constexpr int kRowTilesPerBlock = 4;

template <int DT>
struct Vec8 {
  float v[kVec];
  __device__ __forceinline__ void load(const void *base, int64_t idx) {
    if constexpr (DT == SOPHIA_DTYPE_BF16) {
      u4 w = *reinterpret_cast<const u4 *>(static_cast<const uint16_t *>(base) + idx);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        v[2 * i] = __uint_as_float(w[i] << 16);
        v[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
      }
    } else {
      const f4 *p = reinterpret_cast<const f4 *>(static_cast<const float *>(base) + idx);
      f4 a = p[0], b = p[1];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        v[i] = a[i];
        v[4 + i] = b[i];
      }
    }
  }
  // Outputs are written once and not read back by this kernel: non-temporal
  // stores (64 -> 74 us on the benchmark batch with ordinary stores).  The
  // window loads stay ordinary: neighbouring row tiles re-read 3 rows each.
  __device__ __forceinline__ void store(void *base, int64_t idx) const {
    if constexpr (DT == SOPHIA_DTYPE_BF16) {
      u4 w;
#pragma unroll
      for (int i = 0; i < 4; ++i) w[i] = pack_bf16x2(v[2 * i], v[2 * i + 1]);
      __builtin_nontemporal_store(w, reinterpret_cast<u4 *>(static_cast<uint16_t *>(base) + idx));
    } else {
      f4 *p = reinterpret_cast<f4 *>(static_cast<float *>(base) + idx);
      f4 a, b;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        a[i] = v[i];
        b[i] = v[4 + i];
      }
      __builtin_nontemporal_store(a, p);
      __builtin_nontemporal_store(b, p + 1);
    }
  }
  __device__ __forceinline__ void zero() {
#pragma unroll
    for (int i = 0; i < kVec; ++i) v[i] = 0.f;
  }
};

// Rounds a history value the way the reference does before convolving: the
// cached fp32 history is cast to x's dtype (attention.py:48).
template <int DT>
__device__ __forceinline__ float as_input_dtype(float h) {
  if constexpr (DT == SOPHIA_DTYPE_BF16) return bf16_bits_to_f32(f32_to_bf16_bits(h));
  return h;
}

// Largest s in [0, n) with cu[s] <= row.
__device__ __forceinline__ int find_seq(const int32_t *cu, int n, int64_t row) {
  int lo = 0, hi = n - 1;
  while (lo < hi) {
    int mid = (lo + hi + 1) >> 1;
    if (cu[mid] <= row)
      lo = mid;
    else
      hi = mid - 1;
  }
  return lo;
}

// Packed rows per thread: the whole window of a thread (its rows plus the K-1
// before them) is loaded before any arithmetic, so a thread pays one memory
// round trip.  Eight rows (bf16 and fp32): 57 us on the 12,450 x 6,144 bf16
// batch, against 63 us with 16 rows (137 instead of 105 VGPRs, fewer
// resident waves) and 63 us with 4 (more halo rows per output row).
template <int DT>
constexpr int rows_per_thread() { return 8; }

template <int K, int DT>
__device__ __forceinline__ Vec8<DT> conv_row(const float (&w)[kVec][K], const Vec8<DT> (&win)[K]) {
  Vec8<DT> out;
#pragma unroll
  for (int ci = 0; ci < kVec; ++ci) {
    float acc = 0.f;
#pragma unroll
    for (int j = 0; j < K; ++j) acc = fmaf(w[ci][j], win[j].v[ci], acc);
    out.v[ci] = acc * sigmoid_f(acc);
  }
  return out;
}

template <int K, int DT>
__global__ __launch_bounds__(256) void short_conv_fwd_kernel(
    const void *__restrict__ x, int64_t xs, void *__restrict__ y, int64_t ys,
    const float *__restrict__ weight, const float *__restrict__ conv_state, int n_slots,
    const int32_t *__restrict__ slots, const int32_t *__restrict__ cu, int n_seqs, int64_t total,
    int channels, int read_history) {
  constexpr int R = rows_per_thread<DT>();
  constexpr int HL = K - 1;       // history length
  constexpr int NR = R + HL;      // window rows r0 - HL .. r0 + R - 1
  const int cv = blockIdx.x * kVecsPerBlock + threadIdx.x;
  const int c0 = cv * kVec;
  // threadIdx.y is constant over a wavefront (blockDim.x == 64): r0 and the
  // sequence bookkeeping below are wave-uniform and read cu_seqlens through
  // the scalar cache, off the vector-memory counter the window loads use.
  const int ty = __builtin_amdgcn_readfirstlane(threadIdx.y);
  const int64_t r0 = (static_cast<int64_t>(blockIdx.y) * kRowTilesPerBlock + ty) * R;
  if (c0 >= channels || r0 >= total) return;
  const int64_t r1 = imin64(r0 + R, total);
  // The window is loaded first, before the sequence lookup (whose scalar
  // loads are a chain of dependent round trips); window rows are clamped into
  // [0, total) and are used only when the whole window lies in one sequence.
  Vec8<DT> win[NR];
#pragma unroll
  for (int j = 0; j < NR; ++j) win[j].load(x, iclamp64(r0 - HL + j, 0, total - 1) * xs + c0);
  float w[kVec][K];
#pragma unroll
  for (int i = 0; i < kVec; ++i)
#pragma unroll
    for (int j = 0; j < K; ++j) w[i][j] = weight[static_cast<int64_t>(c0 + i) * K + j];
  // Offsets are clamped to [0, total] and made monotone, so malformed
  // cu_seqlens can never move a read or write outside x, y or conv_state;
  // rows outside every sequence are left untouched.
  int s = find_seq(cu, n_seqs, r0);
  int64_t seq_start = 0, seq_end = 0;
  auto bounds = [&](int seq) {
    seq_start = iclamp64(cu[seq], 0, total);
    seq_end = iclamp64(cu[seq + 1], seq_start, total);
  };
  bounds(s);

  if (r0 - HL >= seq_start && r1 <= seq_end) {
    // Fast path (almost every thread of a long-sequence batch): the window
    // lies inside one sequence.
#pragma unroll
    for (int i = 0; i < R; ++i) {
      if (r0 + i >= r1) break;
      Vec8<DT> taps[K];
#pragma unroll
      for (int j = 0; j < K; ++j) taps[j] = win[i + j];
      conv_row<K, DT>(w, taps).store(y, (r0 + i) * ys + c0);
    }
    return;
  }
  // General path: rows near a sequence start (history or zeros before it) or
  // windows that span several sequences.  Taps are reloaded per row.
  for (int64_t r = r0; r < r1; ++r) {
    while (r >= seq_end && s + 1 < n_seqs) bounds(++s);
    if (r < seq_start || r >= seq_end) continue;
    const float *hist = nullptr;
    if (HL > 0 && r - seq_start < HL && read_history && conv_state != nullptr) {
      const int slot = slots ? slots[s] : s;
      if (slot >= 0 && slot < n_slots) hist = conv_state + static_cast<int64_t>(slot) * channels * HL;
    }
    Vec8<DT> taps[K];
#pragma unroll
    for (int j = 0; j < K; ++j) {
      const int64_t tau = r - HL + j;      // taps[K-1] is the current row
      if (tau >= seq_start) {
        taps[j].load(x, tau * xs + c0);
      } else if (hist != nullptr) {
#pragma unroll
        for (int ci = 0; ci < kVec; ++ci)
          taps[j].v[ci] = as_input_dtype<DT>(hist[static_cast<int64_t>(c0 + ci) * HL + HL + (tau - seq_start)]);
      } else {
        taps[j].zero();
      }
    }
    conv_row<K, DT>(w, taps).store(y, r * ys + c0);
  }
}

// conv_state[slot(s)] <- last K-1 samples of cat(history, x_s).  Runs after
// short_conv_fwd_kernel on the same stream, so the old history has been read.
template <int K, int DT>
__global__ __launch_bounds__(256) void short_conv_history_kernel(
    const void *__restrict__ x, int64_t xs, float *__restrict__ conv_state, int n_slots,
    const int32_t *__restrict__ slots, const int32_t *__restrict__ cu, int n_seqs, int64_t total,
    int channels, int read_history) {
  const int cv = blockIdx.x * blockDim.x + threadIdx.x;
  const int s = blockIdx.y;
  const int c0 = cv * kVec;
  if (c0 >= channels || s >= n_seqs) return;
  const int64_t start = iclamp64(cu[s], 0, total);
  const int64_t end = iclamp64(cu[s + 1], start, total);
  const int slot = slots ? slots[s] : s;
  if (slot < 0 || slot >= n_slots) return;
  float *hist = conv_state + static_cast<int64_t>(slot) * channels * (K - 1);
  float nh[kVec][K - 1];
#pragma unroll
  for (int j = 0; j < K - 1; ++j) {
    const int64_t tau = end - (K - 1) + j;
    if (tau >= start) {
      Vec8<DT> v;
      v.load(x, tau * xs + c0);
#pragma unroll
      for (int i = 0; i < kVec; ++i) nh[i][j] = v.v[i];
    } else {
      const int idx = (K - 1) + static_cast<int>(tau - start);
#pragma unroll
      for (int i = 0; i < kVec; ++i)
        nh[i][j] = read_history
                       ? as_input_dtype<DT>(hist[static_cast<int64_t>(c0 + i) * (K - 1) + idx])
                       : 0.f;
    }
  }
#pragma unroll
  for (int i = 0; i < kVec; ++i)
#pragma unroll
    for (int j = 0; j < K - 1; ++j) hist[static_cast<int64_t>(c0 + i) * (K - 1) + j] = nh[i][j];
}

// One token per sequence: read history, convolve, write the shifted history.
template <int K, int DT>
__global__ __launch_bounds__(256) void short_conv_step_kernel(
    const void *__restrict__ x, int64_t xs, void *__restrict__ y, int64_t ys,
    const float *__restrict__ weight, float *__restrict__ conv_state, int n_slots,
    const int32_t *__restrict__ slots, int batch, int channels, int read_history) {
  const int cv = blockIdx.x * blockDim.x + threadIdx.x;
  const int b = blockIdx.y;
  const int c0 = cv * kVec;
  if (c0 >= channels || b >= batch) return;
  const int slot = slots ? slots[b] : b;
  const bool has_slot = slot >= 0 && slot < n_slots;
  if (!has_slot) read_history = 0;
  float *hist = conv_state + static_cast<int64_t>(has_slot ? slot : 0) * channels * (K - 1);
  Vec8<DT> cur;
  cur.load(x, static_cast<int64_t>(b) * xs + c0);
  float h[kVec][K > 1 ? K - 1 : 1];
  if constexpr (K > 1) {
    if (read_history) {
      // 8 channels x (K-1) fp32 history values are contiguous.
      const float *hp = hist + static_cast<int64_t>(c0) * (K - 1);
#pragma unroll
      for (int i = 0; i < kVec; ++i)
#pragma unroll
        for (int j = 0; j < K - 1; ++j) h[i][j] = as_input_dtype<DT>(hp[i * (K - 1) + j]);
    } else {
#pragma unroll
      for (int i = 0; i < kVec; ++i)
#pragma unroll
        for (int j = 0; j < K - 1; ++j) h[i][j] = 0.f;
    }
  }
  Vec8<DT> out;
#pragma unroll
  for (int i = 0; i < kVec; ++i) {
    float acc = weight[static_cast<int64_t>(c0 + i) * K + (K - 1)] * cur.v[i];
#pragma unroll
    for (int j = 0; j < K - 1; ++j)
      acc = fmaf(weight[static_cast<int64_t>(c0 + i) * K + j], h[i][j], acc);
    out.v[i] = acc * sigmoid_f(acc);
  }
  out.store(y, static_cast<int64_t>(b) * ys + c0);
  if (!has_slot) return;
  if constexpr (K > 1) {
    float *hp = hist + static_cast<int64_t>(c0) * (K - 1);
#pragma unroll
    for (int i = 0; i < kVec; ++i) {
#pragma unroll
      for (int j = 0; j + 1 < K - 1; ++j) hp[i * (K - 1) + j] = h[i][j + 1];
      hp[i * (K - 1) + (K - 2)] = cur.v[i];
    }
  }
}

template <int K, int DT>
int launch_fwd(const void *x, int64_t xs, void *y, int64_t ys, const float *w, float *state,
               int n_slots, const int32_t *slots, const int32_t *cu, int n, int64_t total, int channels,
               int read_history, int write_history, hipStream_t st) {
  const int nvec = channels / kVec;
  dim3 block(kVecsPerBlock, kRowTilesPerBlock);
  constexpr int R = rows_per_thread<DT>();
  const int64_t row_tiles = (total + R - 1) / R;
  dim3 grid((nvec + kVecsPerBlock - 1) / kVecsPerBlock,
            static_cast<unsigned>((row_tiles + kRowTilesPerBlock - 1) / kRowTilesPerBlock));
  if (total > 0) {
    hipLaunchKernelGGL((short_conv_fwd_kernel<K, DT>), grid, block, 0, st, x, xs, y, ys, w, state,
                       n_slots, slots, cu, n, total, channels, read_history && state != nullptr);
    int rc = check_launch("short_conv_fwd");
    if (rc) return rc;
  }
  if constexpr (K > 1) {
    if (write_history && state != nullptr && n > 0) {
      dim3 g2((nvec + 255) / 256, n);
      hipLaunchKernelGGL((short_conv_history_kernel<K, DT>), g2, dim3(256), 0, st, x, xs, state,
                         n_slots, slots, cu, n, total, channels, read_history);
      return check_launch("short_conv_history");
    }
  }
  return SOPHIA_OK;
}

template <int K, int DT>
int launch_step(const void *x, int64_t xs, void *y, int64_t ys, const float *w, float *state,
                int n_slots, const int32_t *slots, int batch, int channels, int read_history, hipStream_t st) {
  const int nvec = channels / kVec;
  dim3 grid((nvec + 255) / 256, batch);
  hipLaunchKernelGGL((short_conv_step_kernel<K, DT>), grid, dim3(256), 0, st, x, xs, y, ys, w,
                     state, n_slots, slots, batch, channels, read_history);
  return check_launch("short_conv_step");
}

template <int DT>
int dispatch_fwd(int K, const void *x, int64_t xs, void *y, int64_t ys, const float *w,
                 float *state, int ns, const int32_t *slots, const int32_t *cu, int n, int64_t total,
                 int channels, int rh, int wh, hipStream_t st) {
  switch (K) {
    case 1: return launch_fwd<1, DT>(x, xs, y, ys, w, state, ns, slots, cu, n, total, channels, rh, wh, st);
    case 2: return launch_fwd<2, DT>(x, xs, y, ys, w, state, ns, slots, cu, n, total, channels, rh, wh, st);
    case 3: return launch_fwd<3, DT>(x, xs, y, ys, w, state, ns, slots, cu, n, total, channels, rh, wh, st);
    case 4: return launch_fwd<4, DT>(x, xs, y, ys, w, state, ns, slots, cu, n, total, channels, rh, wh, st);
  }
  return set_error(SOPHIA_ERR_INVALID, "short_conv: kernel_size %d not in 1..4", K);
}

template <int DT>
int dispatch_step(int K, const void *x, int64_t xs, void *y, int64_t ys, const float *w,
                  float *state, int ns, const int32_t *slots, int batch, int channels, int rh,
                  hipStream_t st) {
  switch (K) {
    case 2: return launch_step<2, DT>(x, xs, y, ys, w, state, ns, slots, batch, channels, rh, st);
    case 3: return launch_step<3, DT>(x, xs, y, ys, w, state, ns, slots, batch, channels, rh, st);
    case 4: return launch_step<4, DT>(x, xs, y, ys, w, state, ns, slots, batch, channels, rh, st);
  }
  return set_error(SOPHIA_ERR_INVALID, "short_conv_step: kernel_size %d not in 2..4", K);
}

// ---- backward (training) ------------------------------------------------------
// With z[u] = sum_j w[j] X[u - (K-1) + j] (X = cat(history, x) of u's
// sequence) and y = silu(z): dz[u] = dy[u] silu'(z[u]), silu' = s (1 + z (1 - s)),
// s = sigmoid(z);  dx[p] = sum_j w[j] dz[p + (K-1) - j] over rows of p's own
// sequence;  dw[j] = sum_u dz[u] X[u - (K-1) + j] (history samples included).
// z is recomputed from x (never stored).  A thread owns 4 channels and a row
// group of kBTiles tiles of kBRows rows: per tile it forms dz for the tile's
// rows and the K-1 after them, writes dx of the tile's rows and adds the
// tile's rows to its dw partial; one partial per (row group, channel) is
// summed over row groups in a fixed order by a second kernel (deterministic).
constexpr int kBVec = 4;
constexpr int kBRows = 8;
constexpr int kBTiles = 16;
constexpr int kBLanes = 64;
constexpr int kBGroups = 4;
constexpr int kBGroupRows = kBRows * kBTiles;

template <int DT>
struct Vec4 {
  float v[kBVec];
  __device__ __forceinline__ void load(const void *base, int64_t idx) {
    if constexpr (DT == SOPHIA_DTYPE_BF16) {
      const u2 w = *reinterpret_cast<const u2 *>(static_cast<const uint16_t *>(base) + idx);
      v[0] = __uint_as_float(w[0] << 16);
      v[1] = __uint_as_float(w[0] & 0xffff0000u);
      v[2] = __uint_as_float(w[1] << 16);
      v[3] = __uint_as_float(w[1] & 0xffff0000u);
    } else {
      const f4 a = *reinterpret_cast<const f4 *>(static_cast<const float *>(base) + idx);
#pragma unroll
      for (int i = 0; i < 4; ++i) v[i] = a[i];
    }
  }
  __device__ __forceinline__ void store(void *base, int64_t idx) const {
    if constexpr (DT == SOPHIA_DTYPE_BF16) {
      *reinterpret_cast<u2 *>(static_cast<uint16_t *>(base) + idx) =
          u2{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
    } else {
      *reinterpret_cast<f4 *>(static_cast<float *>(base) + idx) = f4{v[0], v[1], v[2], v[3]};
    }
  }
};

struct ConvBwdArgs {
  const void *x;
  int64_t xs;
  const void *dy;
  int64_t dys;
  void *dx;
  int64_t dxs;
  const float *weight;
  const float *conv_state;
  int n_slots;
  const int32_t *slots;
  const int32_t *cu;
  int n_seqs;
  int64_t total;
  int channels;
  int read_history;
  float *dw_part;   // [row groups][channels][K]
  float *dw;        // [channels][K]
  int n_groups;
};

template <int K, int DT>
__global__ __launch_bounds__(256) void short_conv_bwd_kernel(ConvBwdArgs a) {
  constexpr int HL = K - 1;
  constexpr int R = kBRows;
  constexpr int NZ = R + HL;   // dz rows of a tile: its R rows and the HL after them
  const int c0 = (blockIdx.x * kBLanes + threadIdx.x) * kBVec;
  const int grp = blockIdx.y * kBGroups + __builtin_amdgcn_readfirstlane(threadIdx.y);
  if (c0 >= a.channels || grp >= a.n_groups) return;
  const int64_t g0 = static_cast<int64_t>(grp) * kBGroupRows;
  float w[kBVec][K];
#pragma unroll
  for (int i = 0; i < kBVec; ++i)
#pragma unroll
    for (int j = 0; j < K; ++j) w[i][j] = a.weight[static_cast<int64_t>(c0 + i) * K + j];
  float dw[kBVec][K];
#pragma unroll
  for (int i = 0; i < kBVec; ++i)
#pragma unroll
    for (int j = 0; j < K; ++j) dw[i][j] = 0.f;
  // Running sequence bounds (offsets clamped into [0, total] and monotone).
  int s = find_seq(a.cu, a.n_seqs, g0);
  int64_t seq_start = 0, seq_end = 0;
  auto bounds = [&](int seq) {
    seq_start = iclamp64(a.cu[seq], 0, a.total);
    seq_end = iclamp64(a.cu[seq + 1], seq_start, a.total);
  };
  bounds(s);
  for (int tile = 0; tile < kBTiles; ++tile) {
    const int64_t r0 = g0 + static_cast<int64_t>(tile) * R;
    if (r0 >= a.total) break;
    float dz[NZ][kBVec];
    int zs[NZ];   // sequence of row r0 + i, -1 outside every sequence
    int ss = s;
    int64_t st = seq_start, en = seq_end;
#pragma unroll
    for (int i = 0; i < NZ; ++i) {
      const int64_t u = r0 + i;
#pragma unroll
      for (int ci = 0; ci < kBVec; ++ci) dz[i][ci] = 0.f;
      zs[i] = -1;
      if (u >= a.total) continue;
      while (u >= en && ss + 1 < a.n_seqs) {
        ++ss;
        st = iclamp64(a.cu[ss], 0, a.total);
        en = iclamp64(a.cu[ss + 1], st, a.total);
      }
      if (u < st || u >= en) continue;
      zs[i] = ss;
      const float *hist = nullptr;
      if (HL > 0 && u - st < HL && a.read_history && a.conv_state != nullptr) {
        const int slot = a.slots ? a.slots[ss] : ss;
        if (slot >= 0 && slot < a.n_slots) hist = a.conv_state + static_cast<int64_t>(slot) * a.channels * HL;
      }
      float tap[K][kBVec];
#pragma unroll
      for (int j = 0; j < K; ++j) {
        const int64_t p = u - HL + j;
        if (p >= st) {
          Vec4<DT> xv;
          xv.load(a.x, p * a.xs + c0);
#pragma unroll
          for (int ci = 0; ci < kBVec; ++ci) tap[j][ci] = xv.v[ci];
        } else {
#pragma unroll
          for (int ci = 0; ci < kBVec; ++ci)
            tap[j][ci] = hist ? as_input_dtype<DT>(hist[static_cast<int64_t>(c0 + ci) * HL + HL + (p - st)]) : 0.f;
        }
      }
      Vec4<DT> g;
      g.load(a.dy, u * a.dys + c0);
#pragma unroll
      for (int ci = 0; ci < kBVec; ++ci) {
        float z = 0.f;
#pragma unroll
        for (int j = 0; j < K; ++j) z = fmaf(w[ci][j], tap[j][ci], z);
        const float sg = sigmoid_f(z);
        dz[i][ci] = g.v[ci] * sg * (1.f + z * (1.f - sg));
      }
      if (i < R) {
#pragma unroll
        for (int ci = 0; ci < kBVec; ++ci)
#pragma unroll
          for (int j = 0; j < K; ++j) dw[ci][j] = fmaf(dz[i][ci], tap[j][ci], dw[ci][j]);
      }
    }
#pragma unroll
    for (int i = 0; i < R; ++i) {
      const int64_t t = r0 + i;
      if (t >= a.total) break;
      Vec4<DT> out;
#pragma unroll
      for (int ci = 0; ci < kBVec; ++ci) {
        float acc = 0.f;
        if (zs[i] >= 0) {
#pragma unroll
          for (int j = 0; j < K; ++j)
            if (zs[i + HL - j] == zs[i]) acc = fmaf(w[ci][j], dz[i + HL - j][ci], acc);
        }
        out.v[ci] = acc;   // rows outside every sequence get zero
      }
      out.store(a.dx, t * a.dxs + c0);
    }
    // the running bounds follow the first row of the next tile
    const int64_t nxt = r0 + R;
    while (nxt >= seq_end && s + 1 < a.n_seqs) bounds(++s);
  }
#pragma unroll
  for (int ci = 0; ci < kBVec; ++ci)
#pragma unroll
    for (int j = 0; j < K; ++j) a.dw_part[(static_cast<int64_t>(grp) * a.channels + c0 + ci) * K + j] = dw[ci][j];
}

// dw[c][j] = sum over row groups (in order) of the partials.
template <int K>
__global__ __launch_bounds__(256) void short_conv_dw_reduce_kernel(ConvBwdArgs a) {
  const int64_t e = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (e >= static_cast<int64_t>(a.channels) * K) return;
  float acc = 0.f;
  for (int gi = 0; gi < a.n_groups; ++gi) acc += a.dw_part[static_cast<int64_t>(gi) * a.channels * K + e];
  a.dw[e] = acc;
}

inline int conv_bwd_groups(int64_t total) { return static_cast<int>((total + kBGroupRows - 1) / kBGroupRows); }

template <int K, int DT>
int launch_bwd(const ConvBwdArgs &a, hipStream_t st) {
  if (a.total > 0) {
    dim3 block(kBLanes, kBGroups);
    dim3 grid((a.channels / kBVec + kBLanes - 1) / kBLanes, (a.n_groups + kBGroups - 1) / kBGroups);
    hipLaunchKernelGGL((short_conv_bwd_kernel<K, DT>), grid, block, 0, st, a);
    if (const int rc = check_launch("short_conv_bwd")) return rc;
  }
  const int64_t n = static_cast<int64_t>(a.channels) * K;
  hipLaunchKernelGGL((short_conv_dw_reduce_kernel<K>), dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0, st,
                     a);
  return check_launch("short_conv_dw_reduce");
}

template <int DT>
int dispatch_bwd(int K, const ConvBwdArgs &a, hipStream_t st) {
  switch (K) {
    case 1: return launch_bwd<1, DT>(a, st);
    case 2: return launch_bwd<2, DT>(a, st);
    case 3: return launch_bwd<3, DT>(a, st);
    case 4: return launch_bwd<4, DT>(a, st);
  }
  return set_error(SOPHIA_ERR_INVALID, "short_conv_bwd: kernel_size %d not in 1..4", K);
}

}  // namespace
}  // namespace sophia

using namespace sophia;

extern "C" int sophia_short_conv_fwd(const void *x, int64_t x_row_stride, void *y,
                                     int64_t y_row_stride, int dtype, const float *weight,
                                     float *conv_state, int n_state_slots,
                                     const int32_t *state_slots, const int32_t *cu_seqlens, int n_seqs, int64_t total_tokens,
                                     int channels, int kernel_size, int read_history,
                                     int write_history, void *stream) {
  SOPHIA_REQUIRE(dtype == SOPHIA_DTYPE_F32 || dtype == SOPHIA_DTYPE_BF16,
                 "short_conv_fwd: dtype %d not supported", dtype);
  SOPHIA_REQUIRE(channels > 0 && channels % kVec == 0,
                 "short_conv_fwd: channels (%d) must be a positive multiple of %d", channels, kVec);
  SOPHIA_REQUIRE(n_seqs > 0 && total_tokens >= 0, "short_conv_fwd: bad n_seqs/total_tokens");
  SOPHIA_REQUIRE(kernel_size >= 1 && kernel_size <= 4, "short_conv_fwd: kernel_size must be 1..4");
  SOPHIA_REQUIRE(weight && cu_seqlens && (total_tokens == 0 || (x && y)),
                 "short_conv_fwd: NULL pointer");
  SOPHIA_REQUIRE(x_row_stride >= channels && y_row_stride >= channels,
                 "short_conv_fwd: row stride smaller than channels");
  SOPHIA_REQUIRE(x_row_stride % kVec == 0 && y_row_stride % kVec == 0,
                 "short_conv_fwd: row strides must be multiples of %d", kVec);
  SOPHIA_REQUIRE(((uintptr_t)x % 16) == 0 && ((uintptr_t)y % 16) == 0,
                 "short_conv_fwd: x and y must be 16-byte aligned");
  SOPHIA_REQUIRE(!(read_history || write_history) || conv_state || kernel_size == 1,
                 "short_conv_fwd: history requested without conv_state");
  SOPHIA_REQUIRE(conv_state == nullptr || n_state_slots >= 0,
                 "short_conv_fwd: n_state_slots must be >= 0");
  SOPHIA_REQUIRE(total_tokens / 32 < 65535, "short_conv_fwd: too many tokens for one launch");
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == SOPHIA_DTYPE_BF16)
    return dispatch_fwd<SOPHIA_DTYPE_BF16>(kernel_size, x, x_row_stride, y, y_row_stride, weight,
                                           conv_state, n_state_slots, state_slots, cu_seqlens,
                                           n_seqs, total_tokens, channels, read_history,
                                           write_history, st);
  return dispatch_fwd<SOPHIA_DTYPE_F32>(kernel_size, x, x_row_stride, y, y_row_stride, weight,
                                        conv_state, n_state_slots, state_slots, cu_seqlens, n_seqs,
                                        total_tokens, channels, read_history, write_history, st);
}

extern "C" int sophia_short_conv_step(const void *x, int64_t x_row_stride, void *y,
                                      int64_t y_row_stride, int dtype, const float *weight,
                                      float *conv_state, int n_state_slots,
                                      const int32_t *state_slots, int batch,
                                      int channels, int kernel_size, int read_history,
                                      void *stream) {
  SOPHIA_REQUIRE(dtype == SOPHIA_DTYPE_F32 || dtype == SOPHIA_DTYPE_BF16,
                 "short_conv_step: dtype %d not supported", dtype);
  SOPHIA_REQUIRE(channels > 0 && channels % kVec == 0,
                 "short_conv_step: channels (%d) must be a positive multiple of %d", channels, kVec);
  SOPHIA_REQUIRE(batch > 0 && batch <= 65535, "short_conv_step: batch must be 1..65535");
  SOPHIA_REQUIRE(kernel_size >= 2 && kernel_size <= 4, "short_conv_step: kernel_size must be 2..4");
  SOPHIA_REQUIRE(x && y && weight && conv_state, "short_conv_step: NULL pointer");
  SOPHIA_REQUIRE(x_row_stride >= channels && y_row_stride >= channels &&
                     x_row_stride % kVec == 0 && y_row_stride % kVec == 0,
                 "short_conv_step: bad row strides");
  SOPHIA_REQUIRE(((uintptr_t)x % 16) == 0 && ((uintptr_t)y % 16) == 0,
                 "short_conv_step: x and y must be 16-byte aligned");
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == SOPHIA_DTYPE_BF16)
    return dispatch_step<SOPHIA_DTYPE_BF16>(kernel_size, x, x_row_stride, y, y_row_stride, weight,
                                            conv_state, n_state_slots, state_slots, batch,
                                            channels, read_history, st);
  return dispatch_step<SOPHIA_DTYPE_F32>(kernel_size, x, x_row_stride, y, y_row_stride, weight,
                                         conv_state, n_state_slots, state_slots, batch, channels,
                                         read_history, st);
}

extern "C" size_t sophia_short_conv_bwd_workspace_size(int64_t total_tokens, int channels, int kernel_size) {
  if (total_tokens < 0 || channels <= 0 || kernel_size < 1 || kernel_size > 4) return 0;
  const size_t groups = static_cast<size_t>(conv_bwd_groups(total_tokens));
  return (groups > 0 ? groups : 1) * static_cast<size_t>(channels) * kernel_size * sizeof(float);
}

extern "C" int sophia_short_conv_bwd(const void *x, int64_t x_row_stride, const void *dy, int64_t dy_row_stride,
                                     void *dx, int64_t dx_row_stride, int dtype, const float *weight,
                                     const float *conv_state, int n_state_slots, const int32_t *state_slots,
                                     const int32_t *cu_seqlens, int n_seqs, int64_t total_tokens, int channels,
                                     int kernel_size, int read_history, float *dweight, void *workspace,
                                     size_t workspace_bytes, void *stream) {
  SOPHIA_REQUIRE(dtype == SOPHIA_DTYPE_F32 || dtype == SOPHIA_DTYPE_BF16,
                 "short_conv_bwd: dtype %d not supported", dtype);
  SOPHIA_REQUIRE(channels > 0 && channels % kBVec == 0,
                 "short_conv_bwd: channels (%d) must be a positive multiple of %d", channels, kBVec);
  SOPHIA_REQUIRE(n_seqs > 0 && total_tokens >= 0 && total_tokens <= 0x7fffffffLL,
                 "short_conv_bwd: bad n_seqs/total_tokens");
  SOPHIA_REQUIRE(kernel_size >= 1 && kernel_size <= 4, "short_conv_bwd: kernel_size must be 1..4");
  SOPHIA_REQUIRE(weight && cu_seqlens && dweight && workspace && (total_tokens == 0 || (x && dy && dx)),
                 "short_conv_bwd: NULL pointer");
  SOPHIA_REQUIRE(x_row_stride >= channels && dy_row_stride >= channels && dx_row_stride >= channels,
                 "short_conv_bwd: row stride smaller than channels");
  SOPHIA_REQUIRE(x_row_stride % kBVec == 0 && dy_row_stride % kBVec == 0 && dx_row_stride % kBVec == 0,
                 "short_conv_bwd: row strides must be multiples of %d", kBVec);
  const uintptr_t al = dtype == SOPHIA_DTYPE_BF16 ? 8 : 16;
  SOPHIA_REQUIRE(((uintptr_t)x % al) == 0 && ((uintptr_t)dy % al) == 0 && ((uintptr_t)dx % al) == 0,
                 "short_conv_bwd: x, dy and dx must be aligned to 4 elements");
  SOPHIA_REQUIRE(!read_history || conv_state || kernel_size == 1, "short_conv_bwd: history requested without conv_state");
  SOPHIA_REQUIRE(conv_state == nullptr || n_state_slots >= 0, "short_conv_bwd: n_state_slots must be >= 0");
  const size_t need = sophia_short_conv_bwd_workspace_size(total_tokens, channels, kernel_size);
  if (workspace_bytes < need)
    return set_error(SOPHIA_ERR_WORKSPACE, "short_conv_bwd: workspace %zu bytes < required %zu", workspace_bytes,
                     need);
  const int groups = conv_bwd_groups(total_tokens);
  SOPHIA_REQUIRE(groups / kBGroups < 65535, "short_conv_bwd: too many tokens for one launch");
  ConvBwdArgs a{x, x_row_stride, dy, dy_row_stride, dx, dx_row_stride, weight, conv_state, n_state_slots,
                state_slots, cu_seqlens, n_seqs, total_tokens, channels, read_history, static_cast<float *>(workspace),
                dweight, groups};
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == SOPHIA_DTYPE_BF16) return dispatch_bwd<SOPHIA_DTYPE_BF16>(kernel_size, a, st);
  return dispatch_bwd<SOPHIA_DTYPE_F32>(kernel_size, a, st);
}
