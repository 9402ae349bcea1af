/* Exhaustive accuracy sweep of the oracle's erf and tanh (oracle/oracle_math.h;
 * the device evaluates the same operation sequence, csrc/kernels/devmath.h)
 * against double-precision libm, over every non-negative binary32 input below
 * the saturation point (erf: |x| < 4, tanh: |x| < 10; above it both return
 * +-1, checked on a stride), plus the odd symmetry f(-x) = -f(x) on a stride
 * of the negatives.  Error is |f(x) - exact| / ulp, ulp = 2^(e - 23) of the
 * exact value's binary32 binade (2^-149 below the normal range).
 * Prints "OK <name> max=<ulp> at=<x> notcr=<fraction>" per function, or FAIL. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "oracle_math.h"

typedef float (*fn32)(float);

static double ulp_of(double t) {
  const float tf = (float)t;
  if (tf == 0.0f || fabsf(tf) < 1.17549435e-38f) return ldexp(1.0, -149);
  return ldexp(1.0, ilogb(tf) - 23);
}

static int sweep(const char* name, fn32 f, double (*ref)(double), uint32_t end, double bound) {
  double mx = 0.0;
  uint32_t arg = 0;
  long notcr = 0, n = 0, asym = 0;
#pragma omp parallel
  {
    double lmx = 0.0;
    uint32_t larg = 0;
#pragma omp for reduction(+ : notcr, n) schedule(dynamic, 64)
    for (uint32_t hi = 0; hi < (end >> 12); ++hi) {
      for (uint32_t lo = 0; lo < 4096u; ++lo) {
        const float x = or_as_float((hi << 12) | lo);
        const double t = ref((double)x);
        const float y = f(x);
        const double e = fabs((double)y - t) / ulp_of(t);
        if (e > lmx) { lmx = e; larg = (hi << 12) | lo; }
        notcr += y != (float)t;
        ++n;
      }
    }
#pragma omp critical
    if (lmx > mx) { mx = lmx; arg = larg; }
  }
  /* saturated range and the odd symmetry, on a stride */
  for (uint64_t u = end; u < 0x7f800000u; u += 997) {
    const float x = or_as_float((uint32_t)u);
    if (f(x) != (float)ref((double)x)) ++asym;
  }
  for (uint64_t u = 0; u < 0x7f800000u; u += 1009) {
    const float x = or_as_float((uint32_t)u);
    const float a = f(x), b = f(-x);
    if (or_as_u32(b) != (or_as_u32(a) ^ 0x80000000u)) ++asym;
  }
  const int ok = mx <= bound && asym == 0;
  printf("%s %s max=%.4f at=%a notcr=%.5f mismatches=%ld\n", ok ? "OK" : "FAIL", name, mx,
         (double)or_as_float(arg), (double)notcr / (double)n, asym);
  return ok ? 0 : 1;
}

int main(int argc, char** argv) {
  const double erf_bound = argc > 1 ? atof(argv[1]) : 0.978;
  const double tanh_bound = argc > 2 ? atof(argv[2]) : 0.5031;
  int rc = sweep("erf", or_erff, erf, 0x40800000u, erf_bound);
  rc |= sweep("tanh", or_tanhf, tanh, 0x41200000u, tanh_bound);
  return rc;
}
