// Unsigned 32-bit division by a run-time-invariant divisor through a
// precomputed multiplier (the round-up method of Granlund & Montgomery,
// "Division by invariant integers using multiplication", PLDI 1994).
//
// For a divisor d in [1, 2^31] pick s = ceil(log2 d) and
//   m = floor(2^32 * (2^s - d) / d) + 1   (fits in 32 bits);
// then for every n < 2^32:  n / d == (umulhi(n, m) + n) >> s,
// with the sum formed in 64 bits.  The offset calculator of the strided
// kernels uses it to turn a linear element index into per-dimension
// coordinates (the role of IntDivider<unsigned> in the reference,
// torch_supa/csrc/aten/ops/kernels/elementwise/IntegerDivider.cuh:82-128).
// Pinned by tests/test_divmod.py, which checks it against exact integer
// division on edge divisors and dividends.
#pragma once

#include <stdint.h>

#if defined(__HIPCC__)
#define SA_HD __host__ __device__ __forceinline__
#else
#define SA_HD inline
#endif

namespace sa {

struct FastDiv {
  uint32_t d;
  uint32_t m;
  uint32_t s;

  FastDiv() : d(1), m(1), s(0) {}
  explicit FastDiv(uint32_t div) : d(div) {
    s = 0;
    while ((uint64_t(1) << s) < div) ++s;
    const uint64_t one = 1;
    m = (uint32_t)(((one << 32) * ((one << s) - div)) / div + 1);
  }
  SA_HD uint32_t div(uint32_t n) const {
#if defined(__HIP_DEVICE_COMPILE__)
    const uint32_t hi = __umulhi(n, m);
#else
    const uint32_t hi = (uint32_t)(((uint64_t)n * m) >> 32);
#endif
    return (uint32_t)(((uint64_t)hi + n) >> s);
  }
  SA_HD void divmod(uint32_t n, uint32_t& q, uint32_t& r) const {
    q = div(n);
    r = n - q * d;
  }
};

}  // namespace sa
