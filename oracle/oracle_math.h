/*
 * TEST INFRASTRUCTURE ONLY -- part of the CPU oracle.  Nothing in the shipped
 * library includes, links or calls this file; only tests/, bench.py's
 * cpu_baseline leg and __graft_entry__.smoke() use the oracle, as the checker.
 *
 * Scalar float32 math primitives of the oracle.  The device kernels evaluate
 * the same polynomials with the same fused-multiply-add sequence, so an
 * elementwise op restated here with these primitives is bit-identical to the
 * device result when both run IEEE binary32 arithmetic with correctly rounded
 * fma, division and ldexp (x86-64 with FMA3 here, gfx950 VALU there).
 *
 * The polynomials were fitted for this project (weighted least squares with
 * Lawson reweighting towards minimax, then rounded to binary32); they do not
 * come from any vendor math library.  Their accuracy against double-precision
 * libm is pinned by tests/test_oracle_math.py:
 *   or_expf  <= 1 ulp,  or_logf <= 1 ulp,  or_erff <= 2 ulp,  or_tanhf <= 2 ulp,
 *   or_expm1f <= 2 ulp, or_log1pf <= 2 ulp.
 *
 * The reductions used by every primitive:
 *   exp:  Cody-Waite split x = k*ln2 + r, |r| <= ln2/2, e^r = 1 + r + r^2 P(r).
 *   log:  x = m * 2^e with m in [sqrt(1/2), sqrt(2)), f = m - 1 (exact),
 *         log1p(f) = f - f^2/2 + f^3 Q(f).
 *   erf:  |x| < 0.921875: erf(x) = x + x P(x^2);
 *         otherwise erf(|x|) = 1 - exp(L(|x|)) with L ~ log(erfc) on
 *         [0.921875, 3.925); 1 beyond.
 *   tanh: |x| < 0.55: x + x^3 T(x^2); otherwise 1 - 2/(exp(2|x|)+1).
 */
#ifndef SUPA_AMD_ORACLE_MATH_H
#define SUPA_AMD_ORACLE_MATH_H

#include <math.h>
#include <stdint.h>
#include <string.h>

static inline float or_as_float(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static inline uint32_t or_as_u32(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

static inline float or_expf(float x) {
  if (isnan(x)) return x;
  x = (x > 89.0f) ? 89.0f : x;
  x = (x < -104.0f) ? -104.0f : x;
  const float k = rintf(x * 1.44269502f);
  float r = fmaf(k, -0.693145751953125f, x);
  r = fmaf(k, -1.42860677e-06f, r);
  float p = 0.0013814599951729178f;
  p = fmaf(p, r, 0.008368715643882751f);
  p = fmaf(p, r, 0.04166838899254799f);
  p = fmaf(p, r, 0.1666652113199234f);
  p = fmaf(p, r, 0.4999999403953552f);
  const float r2 = r * r;
  p = fmaf(p, r2, r);
  p = p + 1.0f;
  return ldexpf(p, (int)k);
}

static inline float or_logf(float x) {
  if (isnan(x)) return x;
  if (x < 0.0f) return NAN;
  if (x == 0.0f) return -INFINITY;
  if (isinf(x)) return x;
  int adj = 0;
  if (x < 1.17549435e-38f) { x = x * 8388608.0f; adj = -23; }
  const uint32_t ix = or_as_u32(x) - 0x3f3504f3u;
  const int e = ((int32_t)ix >> 23) + adj;
  const float f = or_as_float((ix & 0x007fffffu) + 0x3f3504f3u) - 1.0f;
  float q = -0.07634429633617401f;
  q = fmaf(q, f, 0.12761549651622772f);
  q = fmaf(q, f, -0.131601944565773f);
  q = fmaf(q, f, 0.14201761782169342f);
  q = fmaf(q, f, -0.16623356938362122f);
  q = fmaf(q, f, 0.20001226663589478f);
  q = fmaf(q, f, -0.250008225440979f);
  q = fmaf(q, f, 0.3333333134651184f);
  const float f2 = f * f;
  const float y = fmaf(f2, fmaf(f, q, -0.5f), f);
  const float ef = (float)e;
  return fmaf(ef, 0.693145751953125f, fmaf(ef, 1.42860677e-06f, y));
}

static inline float or_erff(float x) {
  const float a = fabsf(x);
  if (a < 0.921875f) {
    const float s = x * x;
    float p = 8.370234718313441e-05f;
    p = fmaf(p, s, -0.0008142741280607879f);
    p = fmaf(p, s, 0.005201036110520363f);
    p = fmaf(p, s, -0.026859400793910027f);
    p = fmaf(p, s, 0.11283695697784424f);
    p = fmaf(p, s, -0.37612634897232056f);
    p = fmaf(p, s, 0.12837916612625122f);
    return fmaf(x, p, x);
  }
  float l = -5.02841658089892e-07f;
  l = fmaf(l, a, -1.4578058653569315e-05f);
  l = fmaf(l, a, 0.00039830547757446766f);
  l = fmaf(l, a, -0.0040588537231087685f);
  l = fmaf(l, a, 0.024906275793910027f);
  l = fmaf(l, a, -0.10802615433931351f);
  l = fmaf(l, a, -0.6335323452949524f);
  l = fmaf(l, a, -1.1294389963150024f);
  l = fmaf(l, a, 0.00016132958990056068f);
  float r = 1.0f - or_expf(l);
  r = (a >= 3.925f) ? 1.0f : r;
  return copysignf(r, x);
}

static inline float or_tanhf(float x) {
  const float a = fabsf(x);
  if (a < 0.55f) {
    const float s = x * x;
    float p = -0.006274243351072073f;
    p = fmaf(p, s, 0.02107168175280094f);
    p = fmaf(p, s, -0.05385231226682663f);
    p = fmaf(p, s, 0.13332585990428925f);
    p = fmaf(p, s, -0.33333316445350647f);
    return fmaf(x * s, p, x);
  }
  const float e = or_expf(a + a);
  const float r = 1.0f - 2.0f / (e + 1.0f);
  return copysignf(r, x);
}

/* gelu 'none' and the normal CDF through log erfc: t = |x| / sqrt(2)
 * (clamped to 3.925), E = erfc(t) = exp(L(t)) with L ~ log(erfc) fitted on
 * [0, 3.925] (degree 11); gelu(x) = x - (x/2) E (x >= 0) or (x/2) E (x < 0),
 * x or -0 once t > 3.925.  The same function as x (1 + erf(x/sqrt2)) / 2
 * without the cancellation of 1 + erf for x << 0: within 1.6 ulp for x >= 0
 * and 9 ulp for x > -2 of double precision, where that form is off by
 * thousands. */
static inline float or_erfc_core(float x) {
  const float tc = fminf(fabsf(x) * 0.70710678118654752f, 3.925f);
  float l = 8.385092797880134e-08f;
  l = fmaf(l, tc, -2.177875103370752e-06f);
  l = fmaf(l, tc, 2.5186680431943387e-05f);
  l = fmaf(l, tc, -0.00016940578643698245f);
  l = fmaf(l, tc, 0.0007112529128789902f);
  l = fmaf(l, tc, -0.001697514788247645f);
  l = fmaf(l, tc, 9.264998516300693e-05f);
  l = fmaf(l, tc, 0.01925601065158844f);
  l = fmaf(l, tc, -0.10283640027046204f);
  l = fmaf(l, tc, -0.6366046667098999f);
  l = fmaf(l, tc, -1.128380537033081f);
  l = fmaf(l, tc, 2.0115285437327657e-08f);
  return or_expf(l);
}
static inline float or_gelu_none(float x) {
  const float t = fabsf(x) * 0.70710678118654752f;
  const float e = or_erfc_core(x);
  const float hx = 0.5f * x;
  float g = (x >= 0.0f) ? fmaf(-hx, e, x) : hx * e;
  g = (t > 3.925f) ? ((x >= 0.0f) ? x : x * 0.0f) : g;
  return g;
}
static inline float or_phif(float x) {
  const float t = fabsf(x) * 0.70710678118654752f;
  const float e = or_erfc_core(x);
  float p = (x >= 0.0f) ? fmaf(-0.5f, e, 1.0f) : 0.5f * e;
  p = (t > 3.925f) ? ((x >= 0.0f) ? 1.0f : 0.0f) : p;
  return isnan(x) ? x : p;
}

/* expm1: the same reduction and polynomial as or_expf (its r + r^2 P(r) is
 * e^r - 1 to 0.85 ulp on |r| <= ln2/2), then 2^k (e^r - 1) + (2^k - 1), or
 * 2^k e^r - 1 once 2^k - 1 is no longer exact (k >= 25). <= 1.5 ulp. */
static inline float or_expm1f(float x) {
  if (isnan(x)) return x;
  x = (x > 89.0f) ? 89.0f : x;
  x = (x < -104.0f) ? -104.0f : x;
  const float k = rintf(x * 1.44269502f);
  float r = fmaf(k, -0.693145751953125f, x);
  r = fmaf(k, -1.42860677e-06f, r);
  float p = 0.0013814599951729178f;
  p = fmaf(p, r, 0.008368715643882751f);
  p = fmaf(p, r, 0.04166838899254799f);
  p = fmaf(p, r, 0.1666652113199234f);
  p = fmaf(p, r, 0.4999999403953552f);
  const float r2 = r * r;
  const float q = fmaf(p, r2, r);
  const int ki = (int)k;
  const float big = ldexpf(q + 1.0f, ki) - 1.0f;
  const float small = ldexpf(q, ki) + (ldexpf(1.0f, ki) - 1.0f);
  return ki >= 25 ? big : small;
}

/* log1p: u = 1 + z rounded, then log(u) + (z - (u - 1)) / u for |z| <= 1
 * (the parenthesis is the exact rounding error of u), log(u) otherwise. */
static inline float or_log1pf(float z) {
  if (isnan(z)) return z;
  if (z < -1.0f) return NAN;
  if (z == -1.0f) return -INFINITY;
  if (isinf(z)) return z;
  const float u = 1.0f + z;
  const float c = (fabsf(z) <= 1.0f) ? z - (u - 1.0f) : 0.0f;
  return or_logf(u) + c / u;
}

#endif
