// Checks the 32-bit splitting of elementwise descriptors (csrc/kernels/
// split32.h) with the limit lowered to small values: over random
// descriptors (1-6 dims, dense, permuted, strided and broadcast operands,
// empty dims) every piece must hold at most `lim` elements, and the pieces
// together must address exactly the (output, input...) element tuples of the
// whole descriptor, each once -- compared against brute-force enumeration.
// A non-zero return of the callback must stop the walk and come back.
#include <algorithm>
#include <cstdint>
#include <cstdio>
#include <random>
#include <tuple>
#include <vector>

#include "split32.h"

using Tuple = std::vector<intptr_t>;

static int esize(int dtype) {
  switch (dtype) {
    case SUPA_AMD_F32: return 4;
    case SUPA_AMD_BF16: return 2;
    case SUPA_AMD_I64: return 8;
    default: return 1;
  }
}

static int64_t numel(const supa_amd_ew_desc& d) {
  int64_t n = 1;
  for (int i = 0; i < d.ndim; ++i) n *= d.sizes[i];
  return n;
}

// every element tuple of d: per operand the byte address of the element
static void enumerate(const supa_amd_ew_desc& d, std::vector<Tuple>& out) {
  const int64_t n = numel(d);
  std::vector<int64_t> idx(std::max(d.ndim, 1), 0);
  for (int64_t e = 0; e < n; ++e) {
    Tuple t;
    for (int k = 0; k < d.noperands; ++k) {
      if (d.op[k].is_scalar) {
        t.push_back(-1);
        continue;
      }
      intptr_t a = reinterpret_cast<intptr_t>(d.op[k].data);
      for (int i = 0; i < d.ndim; ++i) a += idx[i] * d.op[k].strides[i] * esize(d.op[k].dtype);
      t.push_back(a);
    }
    out.push_back(t);
    for (int i = 0; i < d.ndim; ++i) {  // dim 0 fastest
      if (++idx[i] < d.sizes[i]) break;
      idx[i] = 0;
    }
  }
}

int main() {
  std::mt19937_64 rng(2024);
  const int dtypes[] = {SUPA_AMD_F32, SUPA_AMD_BF16, SUPA_AMD_I64, SUPA_AMD_BOOL};
  long cases = 0, pieces_total = 0;
  for (int it = 0; it < 3000; ++it) {
    supa_amd_ew_desc d{};
    d.ndim = 1 + (int)(rng() % 6);
    d.noperands = 1 + (int)(rng() % 4);
    d.common_dtype = SUPA_AMD_F32;
    int64_t total = 1;
    for (int i = 0; i < d.ndim; ++i) {
      d.sizes[i] = (rng() % 23 == 0) ? 0 : 1 + (int64_t)(rng() % 7);
      total *= d.sizes[i];
    }
    if (total > 20000) continue;
    for (int k = 0; k < d.noperands; ++k) {
      supa_amd_operand& o = d.op[k];
      o.dtype = dtypes[rng() % 4];
      o.is_scalar = (k > 0 && rng() % 7 == 0) ? 1 : 0;
      o.data = reinterpret_cast<void*>((intptr_t)(1 + k) << 40);
      // dense in a random dim order, with random gaps and broadcast dims
      std::vector<int> order(d.ndim);
      for (int i = 0; i < d.ndim; ++i) order[i] = i;
      std::shuffle(order.begin(), order.end(), rng);
      int64_t s = 1 + (int64_t)(rng() % 2);
      for (int i : order) {
        o.strides[i] = (k > 0 && rng() % 5 == 0) ? 0 : s;
        s *= std::max<int64_t>(d.sizes[i], 1) + (int64_t)(rng() % 2);
      }
    }
    std::vector<Tuple> ref;
    enumerate(d, ref);
    for (int64_t lim : {1, 2, 3, 7, 13, 64, 1000}) {
      std::vector<Tuple> got;
      int pieces = 0;
      bool too_big = false;
      const int rc = sa::split_32bit(
          d,
          [&](const supa_amd_ew_desc& p) {
            ++pieces;
            if (numel(p) > lim) too_big = true;
            enumerate(p, got);
            return 0;
          },
          esize, lim);
      if (rc != 0 || too_big) {
        std::printf("FAIL case %d lim %lld: rc %d too_big %d\n", it, (long long)lim, rc, (int)too_big);
        return 1;
      }
      std::vector<Tuple> a = ref, b = got;
      std::sort(a.begin(), a.end());
      std::sort(b.begin(), b.end());
      if (a != b) {
        std::printf("FAIL case %d lim %lld: %zu tuples vs %zu expected\n", it, (long long)lim, b.size(), a.size());
        return 1;
      }
      pieces_total += pieces;
      ++cases;
    }
    // early stop: the third piece fails, nothing after it runs
    int calls = 0;
    const int rc = sa::split_32bit(
        d, [&](const supa_amd_ew_desc&) { return ++calls == 3 ? 42 : 0; }, esize, 1);
    const int64_t n = numel(d);
    if ((n >= 3 && (rc != 42 || calls != 3)) || (n > 0 && n < 3 && rc != 0)) {
      std::printf("FAIL case %d: early stop rc %d after %d calls (numel %lld)\n", it, rc, calls, (long long)n);
      return 1;
    }
  }
  std::printf("OK %ld descriptor/limit cases, %ld pieces\n", cases, pieces_total);
  return 0;
}
