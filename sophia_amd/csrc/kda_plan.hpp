// Host-side launch planning of the chunk prefill's state scan: which
// sequences are scanned in which order, over how many value-column slices,
// and which long sequences are cut into segments.  Plain C++17 with no HIP
// dependency, so that it also builds with a host compiler (the CPU tests
// build it under AddressSanitizer and UndefinedBehaviorSanitizer).
//
// Every offset read from the host copy of cu_seqlens is clamped into
// [0, total] and made non-decreasing, as the kernels clamp the device copy:
// malformed offsets give a plan for the clamped batch, never a read or a size
// outside it.
#pragma once

#include <stdint.h>

#include <algorithm>

#include "../../include/sophia_kda.h"

namespace sophia {
namespace plan {

constexpr int kChunk = 64;      // tokens per chunk
constexpr int kOrderMax = 16;   // sequences the host ranks longest first (4-bit order fields)
constexpr int kMaxClasses = 4;  // launch classes of equally sliced chains
constexpr int kSegChunks = 64;  // chunks per segment of the segment-parallel scan
constexpr int kSegSeqMax = 4;   // sequences a segment-parallel scan takes

inline int64_t clamp64(int64_t v, int64_t lo, int64_t hi) { return v < lo ? lo : (v > hi ? hi : v); }

// Chunks of sequence i of a host offset table (clamped as above).
inline int64_t chunks_of(const int32_t *cu_host, int i, int64_t total) {
  const int64_t a = clamp64(cu_host[i], 0, total);
  const int64_t b = clamp64(cu_host[i + 1], a, total);
  return (b - a + kChunk - 1) / kChunk;
}

// Upper bound on the segments of any batch of total_tokens tokens: only a
// sequence of at least 2 kSegChunks chunks is segmented, so the segments
// number at most 1.5 (1 + 1 / (2 kSegChunks - 1)) total / (64 kSegChunks).
inline int64_t max_segments(int64_t total_tokens) {
  if (total_tokens < static_cast<int64_t>(2 * kSegChunks - 1) * kChunk + 1) return 0;
  return 2 * (total_tokens / (static_cast<int64_t>(kSegChunks) * kChunk)) + 2;
}

struct SegPlan {
  bool on = false;
  int run[kSegSeqMax + 1] = {};   // first run segment of sequence s (run[n] = all)
  int cmp[kSegSeqMax + 1] = {};   // first composed segment of sequence s
  int run_splits = 1, cmp_splits = 1;
};

// Segments are used for at most kSegSeqMax sequences with host offsets, when
// their (sequence, head) pairs are too few to fill the chip with 4 slices
// each and the longest has at least 2 kSegChunks chunks.
inline SegPlan plan_segments(const int32_t *cu_host, int n_seqs, int num_heads, int cus, int64_t total,
                             unsigned flags) {
  SegPlan pl;
  if (!cu_host || n_seqs <= 0 || n_seqs > kSegSeqMax || (flags & SOPHIA_KDA_SCAN_NO_SEGMENTS)) return pl;
  if (static_cast<int64_t>(n_seqs) * num_heads * 4 > cus) return pl;
  int64_t chunks[kSegSeqMax] = {}, nmax = 0;
  for (int i = 0; i < n_seqs; ++i) {
    chunks[i] = chunks_of(cu_host, i, total);
    nmax = chunks[i] > nmax ? chunks[i] : nmax;
  }
  if (nmax < 2 * kSegChunks) return pl;
  for (int i = 0; i < n_seqs; ++i) {
    const int64_t nseg = chunks[i] >= 2 * kSegChunks ? (chunks[i] + kSegChunks - 1) / kSegChunks : 1;
    pl.run[i + 1] = pl.run[i] + static_cast<int>(nseg);
    pl.cmp[i + 1] = pl.cmp[i] + static_cast<int>(nseg - 1);
  }
  for (int i = n_seqs + 1; i <= kSegSeqMax; ++i) {
    pl.run[i] = pl.run[n_seqs];
    pl.cmp[i] = pl.cmp[n_seqs];
  }
  if (pl.run[n_seqs] > max_segments(total)) return pl;  // cannot happen (bound above)
  const int64_t run_pairs = static_cast<int64_t>(pl.run[n_seqs]) * num_heads;
  const int64_t cmp_pairs = static_cast<int64_t>(pl.cmp[n_seqs]) * num_heads * 2;
  while (pl.run_splits < 8 && run_pairs * pl.run_splits * 2 <= cus) pl.run_splits *= 2;
  while (pl.cmp_splits < 8 && cmp_pairs * pl.cmp_splits * 2 <= cus) pl.cmp_splits *= 2;
  pl.on = true;
  return pl;
}

// The scan launch.  Every (sequence, head) pair of the batch would get the
// same number of work-groups (slices of the 128 value columns): as many as
// keep every work-group resident at once.  With the host copy of the offsets
// (and at most kOrderMax sequences), sequences are taken longest first, a
// batch whose longest sequence has at least twice the mean number of chunks
// gets twice that number for its longest chains, and shorter chains get fewer
// slices: half for a chain of under 60 % of the longest, a quarter under 30 %
// (at least one).  Measured on one MI355X, the 8 sequences of U[256, 4096]
// tokens (56 chunks at most, 16 heads): 4/4/4/2/2/1/1/1 slices 197 us per
// prefill call, 4 everywhere 206 us, 8 on the longest chain and 4 elsewhere
// 214 us (a slice's step reads the pair's whole -W / Q e^G / Kbar^T / A_qk
// record parts, so more slices per chain cost more in total than they save on
// the chain once the chip is full).
//   order_bits: 4-bit field r = the sequence taken at rank r < n (the
//               identity past n, and for batches without a host plan);
//   class c owns ranks [rank[c], rank[c + 1]) and work-groups [block[c],
//   block[c + 1]); each of its pairs runs on splits[c] work-groups; a class's
//   pairs are padded to a multiple of 8 so that the slices of one pair share
//   an XCD (work-group b runs on XCD b % 8).
struct ScanPlan {
  int n_cls = 1;
  int block[kMaxClasses + 1] = {};
  int rank[kMaxClasses + 1] = {};
  int splits[kMaxClasses] = {1, 1, 1, 1};
  uint64_t order_bits = 0xfedcba9876543210ull;
  int64_t blocks = 0;
};

inline ScanPlan plan_scan(const int32_t *cu_host, int n_seqs, int num_heads, int cus, int64_t total) {
  ScanPlan pl;
  const int64_t pairs = static_cast<int64_t>(n_seqs) * num_heads;
  int top = 1;
  while (top < 8 && pairs * top * 2 <= static_cast<int64_t>(cus)) top *= 2;
  if (!cu_host || n_seqs > kOrderMax) {
    pl.splits[0] = top;
    pl.rank[1] = n_seqs;
    pl.blocks = (pairs + 7) / 8 * 8 * top;
    pl.block[1] = static_cast<int>(pl.blocks);
    return pl;
  }
  int order[kOrderMax];
  int64_t chunks[kOrderMax];
  int64_t nmax = 0, sum = 0;
  for (int i = 0; i < n_seqs; ++i) {
    order[i] = i;
    chunks[i] = chunks_of(cu_host, i, total);
    nmax = chunks[i] > nmax ? chunks[i] : nmax;
    sum += chunks[i];
  }
  if (top < 8 && sum > 0 && nmax * n_seqs >= 2 * sum) top *= 2;
  std::stable_sort(order, order + n_seqs, [&](int a, int b) { return chunks[a] > chunks[b]; });
  for (int r = 0; r < n_seqs; ++r)
    pl.order_bits = (pl.order_bits & ~(15ull << (4 * r))) | (static_cast<uint64_t>(order[r]) << (4 * r));
  int sp[kOrderMax];
  for (int r = 0; r < n_seqs; ++r) {
    const int64_t c = chunks[order[r]];
    int v = top;
    if (10 * c < 6 * nmax) v = top / 2;
    if (10 * c < 3 * nmax) v = top / 4;
    sp[r] = v < 1 ? 1 : v;
  }
  pl.n_cls = 0;
  int64_t block = 0;
  for (int r = 0; r < n_seqs;) {
    int e = r;
    while (e < n_seqs && sp[e] == sp[r]) ++e;
    const int c = pl.n_cls++;
    pl.rank[c] = r;
    pl.block[c] = static_cast<int>(block);
    pl.splits[c] = sp[r];
    block += (static_cast<int64_t>(e - r) * num_heads + 7) / 8 * 8 * sp[r];
    r = e;
  }
  pl.rank[pl.n_cls] = n_seqs;
  pl.block[pl.n_cls] = static_cast<int>(block);
  pl.blocks = block;
  return pl;
}

}  // namespace plan
}  // namespace sophia
