// Chunk index of a multi-tensor table (host fill, device lookup).
//
// A table lists up to kMtaTensors tensors with the prefix sums of their
// chunk counts (chunk_start[0..ntensors], non-decreasing; an empty tensor
// repeats its neighbour's start).  A workgroup's tensor is the last k with
// chunk_start[k] <= blockIdx.  bucket[b] holds that answer for chunk
// b << bucket_shift, and every chunk of the table falls in one of the
// kMtaBuckets buckets, so the lookup is a short forward scan from the
// bucket's entry -- usually none or one step on large tensors -- where a
// bisection of a 40-entry table costs six dependent scalar loads before the
// workgroup's first vector load can issue.  Pinned by tests/test_mta_index.py
// against bisection by brute force.
#pragma once

#include <stdint.h>

#if defined(__HIPCC__)
#define SA_MTA_HD __host__ __device__ __forceinline__
#else
#define SA_MTA_HD inline
#endif

namespace sa {

constexpr int kMtaTensors = 40;
constexpr int kMtaBuckets = 64;
// 32-bit entries: gfx9 scalar loads read whole dwords, so with byte entries
// the compiler fetched a workgroup's entry with a vector load and waited for
// it before the scalar lookups and the first data load could issue.  Over
// c5's 72 tensors the norm partials ran at 77-80 % of the HBM roofline with
// byte entries and at 90-92 % with 32-bit ones (the kernel over one flat
// buffer with no lookup: 91 %).
using MtaBucket = uint32_t;

// Fills tab.bucket / tab.bucket_shift from tab.chunk_start[0..ntensors] and
// the table's chunk count.
template <typename Table>
void mta_index(Table& tab, uint32_t chunks) {
  uint32_t s = 0;
  const uint64_t last = chunks ? chunks - 1u : 0u;
  while ((last >> s) >= (uint64_t)kMtaBuckets) ++s;
  tab.bucket_shift = s;
  int k = 0;
  for (int b = 0; b < kMtaBuckets; ++b) {
    const uint64_t first = (uint64_t)b << s;
    while (k + 1 < tab.ntensors && tab.chunk_start[k + 1] <= first) ++k;
    tab.bucket[b] = (MtaBucket)k;
  }
}

// The last k with chunk_start[k] <= blk, for blk below the table's chunks.
template <typename Table>
SA_MTA_HD int find_tensor(const Table& tab, uint32_t blk) {
  int k = tab.bucket[blk >> tab.bucket_shift];
  while (k + 1 < tab.ntensors && tab.chunk_start[k + 1] <= blk) ++k;
  return k;
}

}  // namespace sa
