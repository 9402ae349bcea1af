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
 * Lawson reweighting towards minimax); they do not come from any vendor math
 * library.  Their accuracy against double-precision libm (exhaustive over
 * every binary32 input for erf and tanh) is pinned by
 * tests/test_oracle_math.py:
 *   or_expf <= 1.01 ulp, or_logf <= 0.94 ulp, or_erff <= 0.978 ulp,
 *   or_tanhf <= 0.5031 ulp, or_expm1f <= 1.5 ulp, or_log1pf <= 2 ulp.
 *
 * The reductions used by every primitive:
 *   exp:  Cody-Waite split x = k*ln2 + r, |r| <= ln2/2, e^r = 1 + r + r^2 P(r).
 *   log:  x = m * 2^e with m in [sqrt(1/2), sqrt(2)), f = m - 1 (exact),
 *         log1p(f) = f - f^2/2 + f^3 Q(f).
 *   erf:  |x| < 0.921875: x + x P(x^2); otherwise 1 - Q(|x| - c), Q ~ erfc
 *         on [0.921875, 2.25) and [2.25, 3.9375); +-1 beyond.
 *   tanh: binary64 core: tanh(a) = m / (m + 2), m = e^{2a} - 1 from
 *         2a = k ln2 + 2s and e^{2s} - 1 = s (2 + s Q(s)); the quotient is
 *         the IEEE binary64 quotient m / (m + 2).
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

/* Only IEEE-specified operations are used below (fma, multiply, add,
 * divide, integer operations on the bits, conversions), so device and oracle
 * agree bit for bit.
 *
 * erf (binary32, <= 0.978 ulp over every input; 1.5 % of results are not
 * correctly rounded).  Three ranges of |x|:
 *   [0, 0.921875):    x + x P(x^2), P of degree 6 (relative error 2^-31
 *                     against erf(x)/x - 1);
 *   [0.921875, 2.25): 1 - M(|x| - 1.5859375), M ~ erfc of degree 9;
 *   [2.25, 3.9375):   1 - T(|x| - 3.09375), T ~ erfc of degree 9 (absolute
 *                     errors 2^-27);
 *   beyond: +-1 (erfc(3.9375) < 2^-25, so erf rounds to 1 there).
 * |x| - c is exact in both erfc ranges (Sterbenz). */
/* Test hook: tests/test_gelu_parity.py builds a separate copy of the oracle
 * with OR_ERF_SCALE defined to 1 +- k 2^-24 (a k-ulp change of erf), to show
 * that its gelu checks detect such a change.  Here it is 1, an exact
 * identity. */
#ifndef OR_ERF_SCALE
#define OR_ERF_SCALE 1.0f
#endif

/* or_erff without the NaN select (the device's sa_erff_nn): the same value
 * for every non-NaN x; gelu uses it. */
static inline float or_erff_nn(float x) {
  const float a = fabsf(x);
  float r;
  if (a < 0.921875f) {
    const float s = x * x;
    float p = 8.370154682779685e-05f;
    p = fmaf(p, s, -0.0008142719161696732f);
    p = fmaf(p, s, 0.005201033782213926f);
    p = fmaf(p, s, -0.026859398931264877f);
    p = fmaf(p, s, 0.11283695697784424f);
    p = fmaf(p, s, -0.37612634897232056f);
    p = fmaf(p, s, 0.12837916612625122f);
    r = fmaf(x, p, x);
  } else {
    float q;
    if (a < 2.25f) {
      const float t = a - 1.5859375f;
      q = -0.001323151052929461f;
      q = fmaf(q, t, 0.0013511608121916652f);
      q = fmaf(q, t, 0.0058217644691467285f);
      q = fmaf(q, t, -0.01616346836090088f);
      q = fmaf(q, t, 0.005730860400944948f);
      q = fmaf(q, t, 0.048972442746162415f);
      q = fmaf(q, t, -0.12256082892417908f);
      q = fmaf(q, t, 0.1446780115365982f);
      q = fmaf(q, t, -0.09122593700885773f);
      q = fmaf(q, t, 0.02490621618926525f);
    } else {
      const float t = a - 3.09375f;
      q = -7.529089998570271e-06f;
      q = fmaf(q, t, 0.00010170548193855211f);
      q = fmaf(q, t, -0.0003080983296968043f);
      q = fmaf(q, t, 0.0005250130197964609f);
      q = fmaf(q, t, -0.0006629122071899474f);
      q = fmaf(q, t, 0.0006516603752970695f);
      q = fmaf(q, t, -0.00047629239270463586f);
      q = fmaf(q, t, 0.00024359175586141646f);
      q = fmaf(q, t, -7.862227357691154e-05f);
      q = fmaf(q, t, 1.2126994079153519e-05f);
      q = (a >= 3.9375f) ? 0.0f : q;  // erf rounds to +-1 beyond
    }
    r = copysignf(1.0f - q, x);
  }
  return r * OR_ERF_SCALE;
}

static inline float or_erff(float x) { return isnan(x) ? x : or_erff_nn(x); }

/* tanh rounds a binary64 core once to binary32, so it is correctly rounded
 * except where the exact value lies within the core's error of a binary32
 * rounding boundary (binary64 fma runs at the binary32 rate on the device).
 *
 * tanh: with a = min(|x|, 9.5) (tanh(9.5) rounds to 1), 2a = k ln2 + 2s,
 * |s| <= ln2/4, k from the 1.5 * 2^52 shifter (the low word of the sum);
 * e^{2s} - 1 = s (2 + s Q(s)), Q of degree 5 (relative error 2^-32.0);
 * m = e^{2a} - 1 = 2^k (e^{2s} - 1) + (2^k - 1), 2^k built from its exponent
 * field, which keeps m's relative accuracy as a -> 0; tanh(a) = m / (m + 2),
 * the binary64 quotient, with x's sign.  The device reaches the same quotient from its hardware
 * reciprocal with one Newton step and one residual correction (exact but for
 * quotients within 2^-97 of a binary64 rounding midpoint). */
static inline double or_hilo(uint32_t hi, uint32_t lo) {
  const uint64_t u = ((uint64_t)hi << 32) | lo;
  double d;
  memcpy(&d, &u, 8);
  return d;
}
static inline uint64_t or_bits64(double d) { uint64_t u; memcpy(&u, &d, 8); return u; }
static inline double or_tanh_quot(float x) {
  const float a = fminf(fabsf(x), 9.5f);
  const double d = (double)a;
  const double kb = fma(d, 2.8853900817779268, 6755399441055744.0);
  const double k = kb - 6755399441055744.0;
  const double s = fma(-k, 0.34657359027997264, d);
  double q = 0.02540272786494247;
  q = fma(q, s, 0.08922027840168137);
  q = fma(q, s, 0.26666846268672123);
  q = fma(q, s, 0.6666617668472024);
  q = fma(q, s, 1.3333333095802695);
  q = fma(q, s, 2.000000017707398);
  const double e = s * fma(s, q, 2.0);
  const int32_t ki = (int32_t)(uint32_t)or_bits64(kb);
  const double p2 = or_hilo((uint32_t)(ki + 1023) << 20, 0);
  const double m = fma(p2, e, p2 - 1.0);
  const double h = m + 2.0;
  return m / h;
}
static inline float or_tanhf(float x) {
  const float r = copysignf((float)or_tanh_quot(x), x);
  return isnan(x) ? x : r;
}
/* gelu('tanh') forward on the device skips the residual correction: its
 * quotient is within 2^-48.5 (relative) of m / h, so its binary32 value is
 * or_tanhf's except where m / h lies that close to a binary32 rounding
 * boundary, where it may be the other neighbour.  This returns that other
 * neighbour when m / h is within 2^-44 (a margin of 2^4.5) of a boundary, and
 * or_tanhf's value otherwise: the device result is one of the two. */
static inline float or_tanhf_fast_alt(float x) {
  const double q = or_tanh_quot(x);
  const float f = (float)q;
  const float lo = (float)(q * (1.0 - 0x1p-44));
  const float hi = (float)(q * (1.0 + 0x1p-44));
  const float r = copysignf(lo != f ? lo : hi, x);
  return isnan(x) ? x : r;
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
