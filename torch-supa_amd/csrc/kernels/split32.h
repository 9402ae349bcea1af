// Splitting of an elementwise descriptor into pieces whose element count
// fits the 32-bit coordinate arithmetic of the N-d kernels.  Plain C++ on the
// descriptor of include/supa_amd.h (no HIP), so the CPU tests can drive it
// with a small limit and check it against brute-force enumeration.
#pragma once

#include <stdint.h>

#include <algorithm>

#include "supa_amd.h"

namespace sa {

constexpr int64_t kSplitLimit = (int64_t(1) << 31) - 1;

// Calls fn(piece) on sub-descriptors covering every element of d exactly
// once, each with at most `lim` elements: the outermost dims are cut (the
// last descriptor dim is the outermost; dim 0 moves fastest), first by
// slicing the outermost dim into runs, and when the inner dims alone exceed
// the limit, by peeling it element by element and recursing.  esize(dtype)
// gives an operand's element size in bytes.  Stops at the first non-zero
// return of fn and returns it.  The reference splits the same way
// (Loops.cuh:100-105, TensorIterator::with_32bit_indexing).
template <typename Fn, typename ESize>
int split_32bit(const supa_amd_ew_desc& d, Fn&& fn, ESize&& esize, int64_t lim = kSplitLimit) {
  int64_t n = 1;
  for (int i = 0; i < d.ndim; ++i) n *= d.sizes[i];
  if (n <= lim) return fn(d);
  const int last = d.ndim - 1;
  int64_t inner = 1;
  for (int i = 0; i < last; ++i) inner *= d.sizes[i];
  const int64_t outer = d.sizes[last];
  if (inner <= lim) {
    const int64_t step = std::max<int64_t>(1, lim / std::max<int64_t>(inner, 1));
    for (int64_t o = 0; o < outer; o += step) {
      supa_amd_ew_desc s = d;
      s.sizes[last] = std::min(step, outer - o);
      for (int k = 0; k < d.noperands; ++k)
        if (!s.op[k].is_scalar)
          s.op[k].data = static_cast<char*>(d.op[k].data) + o * d.op[k].strides[last] * esize(d.op[k].dtype);
      const int rc = fn(s);
      if (rc) return rc;
    }
    return SUPA_AMD_OK;
  }
  for (int64_t o = 0; o < outer; ++o) {
    supa_amd_ew_desc s = d;
    s.ndim = last;
    for (int k = 0; k < d.noperands; ++k)
      if (!s.op[k].is_scalar)
        s.op[k].data = static_cast<char*>(d.op[k].data) + o * d.op[k].strides[last] * esize(d.op[k].dtype);
    const int rc = split_32bit(s, fn, esize, lim);
    if (rc) return rc;
  }
  return SUPA_AMD_OK;
}

}  // namespace sa
