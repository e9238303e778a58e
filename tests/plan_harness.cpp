// CPU driver of the prefill's host launch planners (sophia_amd/csrc/kda_plan.hpp),
// built by tests/test_launch_plan.py with g++ under AddressSanitizer and
// UndefinedBehaviorSanitizer.  Reads one case per line from stdin:
//   scan <n_seqs> <num_heads> <cus> <total> <has_host 0|1> <cu_0> ... <cu_n>
//   seg  <n_seqs> <num_heads> <cus> <total> <flags> <cu_0> ... <cu_n>
// and prints each plan as one JSON object per line.
#include <cinttypes>
#include <cstdio>
#include <cstring>
#include <vector>

#include "../sophia_amd/csrc/kda_plan.hpp"

using namespace sophia::plan;

int main() {
  char kind[8];
  while (std::scanf("%7s", kind) == 1) {
    int n = 0, heads = 0, cus = 0;
    long long total = 0;
    unsigned extra = 0;
    if (std::scanf("%d %d %d %lld %u", &n, &heads, &cus, &total, &extra) != 5) return 2;
    std::vector<int32_t> cu(n > 0 ? n + 1 : 1);
    for (int i = 0; i <= n && n > 0; ++i)
      if (std::scanf("%d", &cu[i]) != 1) return 2;
    if (std::strcmp(kind, "scan") == 0) {
      const ScanPlan p = plan_scan(extra ? cu.data() : nullptr, n, heads, cus, total);
      std::printf("{\"n_cls\": %d, \"blocks\": %" PRId64 ", \"order_bits\": %" PRIu64 ", \"rank\": [", p.n_cls,
                  p.blocks, p.order_bits);
      for (int c = 0; c <= kMaxClasses; ++c) std::printf("%s%d", c ? ", " : "", p.rank[c]);
      std::printf("], \"block\": [");
      for (int c = 0; c <= kMaxClasses; ++c) std::printf("%s%d", c ? ", " : "", p.block[c]);
      std::printf("], \"splits\": [");
      for (int c = 0; c < kMaxClasses; ++c) std::printf("%s%d", c ? ", " : "", p.splits[c]);
      std::printf("]}\n");
    } else {
      const SegPlan p = plan_segments(cu.data(), n, heads, cus, total, extra);
      std::printf("{\"on\": %s, \"run_splits\": %d, \"cmp_splits\": %d, \"max_segments\": %" PRId64 ", \"run\": [",
                  p.on ? "true" : "false", p.run_splits, p.cmp_splits, max_segments(total));
      for (int s = 0; s <= kSegSeqMax; ++s) std::printf("%s%d", s ? ", " : "", p.run[s]);
      std::printf("], \"cmp\": [");
      for (int s = 0; s <= kSegSeqMax; ++s) std::printf("%s%d", s ? ", " : "", p.cmp[s]);
      std::printf("]}\n");
    }
  }
  return 0;
}
