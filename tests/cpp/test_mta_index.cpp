// Checks the bucket index of the multi-tensor tables (csrc/kernels/
// mta_index.h) against bisection of the chunk prefix table, for every block
// of random tables: empty and one-chunk tensors, one huge tensor, full
// 40-tensor tables, and chunk totals up to 2^31 - 1 (there on sampled blocks).
#include <cstdint>
#include <cstdio>
#include <random>
#include <vector>

#include "mta_index.h"

struct Tab {
  uint32_t chunk_start[sa::kMtaTensors + 1];
  int32_t ntensors;
  uint32_t bucket_shift;
  sa::MtaBucket bucket[sa::kMtaBuckets];
};

static int bisect(const Tab& t, uint32_t blk) {
  int lo = 0, hi = t.ntensors - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (t.chunk_start[mid] <= blk) lo = mid;
    else hi = mid - 1;
  }
  return lo;
}

int main() {
  std::mt19937_64 rng(12345);
  long checked = 0;
  for (int trial = 0; trial < 4000; ++trial) {
    Tab t{};
    const int nt = 1 + (int)(rng() % sa::kMtaTensors);
    const int kind = trial % 4;
    uint64_t total = 0;
    std::vector<uint64_t> counts(nt);
    for (int k = 0; k < nt; ++k) {
      uint64_t c;
      if (kind == 0) c = rng() % 3;                                  // empty and tiny
      else if (kind == 1) c = (rng() % 5 == 0) ? 0 : 1 + rng() % 5000;
      else if (kind == 2) c = (k == nt / 2) ? 1 + rng() % 2000000 : rng() % 4;  // one huge
      else c = 1 + rng() % ((1u << 31) / sa::kMtaTensors - 1);        // near the 2^31 limit
      counts[k] = c;
      total += c;
    }
    if (total == 0) counts[0] = total = 1;
    if (total >= (1ull << 31)) continue;
    uint32_t s = 0;
    for (int k = 0; k < nt; ++k) {
      t.chunk_start[k] = s;
      s += (uint32_t)counts[k];
    }
    t.chunk_start[nt] = s;
    t.ntensors = nt;
    sa::mta_index(t, s);
    if ((uint64_t)((s - 1) >> t.bucket_shift) >= (uint64_t)sa::kMtaBuckets) {
      printf("FAIL bucket range trial %d\n", trial);
      return 1;
    }
    auto check = [&](uint32_t blk) {
      if (sa::find_tensor(t, blk) != bisect(t, blk)) {
        printf("FAIL trial %d blk %u: %d vs %d\n", trial, blk, sa::find_tensor(t, blk), bisect(t, blk));
        return false;
      }
      ++checked;
      return true;
    };
    if (s <= 3000000u) {
      for (uint32_t b = 0; b < s; ++b)
        if (!check(b)) return 1;
    } else {
      for (int k = 0; k <= nt; ++k)
        for (int64_t d = -2; d <= 2; ++d) {
          const int64_t b = (int64_t)t.chunk_start[k] + d;
          if (b >= 0 && b < (int64_t)s && !check((uint32_t)b)) return 1;
        }
      for (int r = 0; r < 20000; ++r)
        if (!check((uint32_t)(rng() % s))) return 1;
    }
  }
  printf("OK %ld blocks\n", checked);
  return 0;
}
