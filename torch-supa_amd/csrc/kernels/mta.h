// Multi-tensor apply: the pieces every list kernel shares.
//
// One launch covers up to kMtaTensors tensors.  The tensor table (pointers,
// element counts, chunk prefix sums) travels in the kernel arguments, so a
// launch needs no device-side metadata and no allocation.  Each workgroup
// owns one chunk of one tensor, found through a bucket index of the chunk
// prefix table.
// The reference's counterpart is upstream MultiTensorApply.cuh (kChunkSize
// 65536, 512 threads, ILP 4, <= 110 / 36 tensors per launch).
#pragma once

#include "ew_launch.h"
#include "mta_index.h"

namespace sa {

// One wavefront per workgroup: c5's fused AdamW moved 74 % of peak HBM
// bandwidth with 64-thread workgroups against 71 % with 256 and 70 % with 128.
constexpr int kMtaBlock = 64;
// Elements per workgroup: one 16-byte vector per thread -- the fastest
// measured on MI355X (c5 AdamW at 256 threads: 71 % of HBM peak against 66 %
// with 16384-element chunks).
template <typename T> constexpr int64_t chunk_one() { return (int64_t)kMtaBlock * (16 / (int64_t)sizeof(T)); }

// The [lo, hi) element range of block `blk` within tensor k.
struct MtaRange {
  int k;
  int64_t lo, hi;
};
template <int64_t CHUNK, typename Table>
__device__ __forceinline__ MtaRange mta_range(const Table& tab) {
  MtaRange r;
  r.k = find_tensor(tab, blockIdx.x);
  r.lo = (int64_t)(blockIdx.x - tab.chunk_start[r.k]) * CHUNK;
  const int64_t n = tab.numel[r.k];
  r.hi = r.lo + CHUNK < n ? r.lo + CHUNK : n;
  return r;
}

// Packs tensors [0, ntensors) into tables of at most kMtaTensors non-empty
// tensors and fewer than 2^31 chunks, and launches once per table.
//   fill(tab, slot, i)   copies tensor i's pointers into table slot `slot`
//   launch(tab, chunks)  launches the kernel over one table
// Table must have numel[], chunk_start[], ntensors, bucket[] and
// bucket_shift.  Empty tensors are skipped; a negative numel is an argument
// error.
template <int64_t CHUNK, typename Table, typename Fill, typename Launch>
int mta_for_tables(int32_t ntensors, const int64_t* numel, Fill&& fill, Launch&& launch) {
  int i = 0;
  while (i < ntensors) {
    Table tab{};
    uint32_t chunks = 0;
    int nt = 0;
    while (i < ntensors && nt < kMtaTensors) {
      if (numel[i] < 0) return SUPA_AMD_EINVAL;
      const int64_t c = (numel[i] + CHUNK - 1) / CHUNK;
      if (c > (int64_t)0x7fffffff) return SUPA_AMD_ELAYOUT;
      if ((int64_t)chunks + c > (int64_t)0x7fffffff) break;
      if (numel[i] > 0) {
        const int rc = fill(tab, nt, i);
        if (rc) return rc;
        tab.numel[nt] = numel[i];
        tab.chunk_start[nt] = chunks;
        chunks += (uint32_t)c;
        ++nt;
      }
      ++i;
    }
    tab.chunk_start[nt] = chunks;
    tab.ntensors = nt;
    if (nt == 0) continue;
    mta_index(tab, chunks);
    launch(tab, chunks);
    const int rc = launch_status();
    if (rc) return rc;
  }
  return SUPA_AMD_OK;
}

template <typename F>
int with_mta_storage(int dtype, F&& f) {
  switch (dtype) {
    case SUPA_AMD_F32: return f((float*)nullptr);
    case SUPA_AMD_BF16: return f((bf16*)nullptr);
    case SUPA_AMD_F16: return f((f16*)nullptr);
    case SUPA_AMD_F64: return f((double*)nullptr);
    default: return SUPA_AMD_EDTYPE;
  }
}

}  // namespace sa
