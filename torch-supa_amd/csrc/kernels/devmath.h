// Float32 math primitives of the elementwise kernels.
//
// Own implementations (not the device libm), evaluated with an explicit
// fused-multiply-add sequence and compiled with -ffp-contract=off, so every
// result is reproducible bit for bit by any IEEE machine with correctly
// rounded binary32/binary64 fma, add, multiply, division, rint and ldexp
// (tanh's quotient starts from the hardware reciprocal and is corrected to
// the binary64 quotient; gelu('tanh') forward's uncorrected quotient is the
// one exception, described at sa_tanhf_fast_nn).  Accuracy against
// double-precision math, measured over every binary32 input:
//   sa_expf <= 1.01 ulp, sa_logf <= 0.93 ulp, sa_erff <= 0.978 ulp,
//   sa_tanhf <= 0.5031 ulp, sa_expm1f <= 1.5 ulp, sa_log1pf <= 2 ulp.
// The polynomial coefficients were fitted for this project (weighted least
// squares with Lawson reweighting towards minimax).
//
// Reductions:
//   exp:  x = k ln2 + r (Cody-Waite two-constant split), |r| <= ln2/2,
//         e^r = 1 + r + r^2 P(r), result = ldexp(e^r, k).
//   log:  x = m 2^e, m in [sqrt(1/2), sqrt(2)), f = m - 1 (exact),
//         log(x) = e ln2 + f - f^2/2 + f^3 Q(f).
//   erf:  |x| < 0.921875: x + x P(x^2); otherwise 1 - Q(|x| - c), Q ~ erfc
//         on [0.921875, 2.25) and on [2.25, 3.9375); +-1 beyond.
//   tanh: binary64 core rounded once: tanh(a) = m / (m + 2), m = e^{2a} - 1
//         from 2a = k ln2 + 2s and e^{2s} - 1 = s (2 + s Q(s)); the quotient
//         m / (m + 2) as the correctly rounded binary64 quotient.
// Binary64 fma runs at the binary32 rate on gfx950, so tanh's binary64 core
// costs about what a binary32 evaluation with the same number of terms does,
// and rounds correctly except within 2^-31.7 of a binary32 rounding boundary
// (0.008 % of inputs).
#pragma once

#include <hip/hip_runtime.h>

namespace sa {

// Binary64 polynomial coefficients of the tanh core, highest degree first.
// They live in constant memory (not const-qualified, so the compiler loads
// them instead of folding them): a kernel reads them once into SGPRs, where
// every v_fma_f64 can take them as its scalar operand; as 64-bit literals
// each use would cost two v_mov_b32 into VGPRs (gfx9 VOP3 takes no literal
// operand).
__constant__ inline double kTanhQ[6] = {
    0.02540272786494247, 0.08922027840168137, 0.26666846268672123,
    0.6666617668472024, 1.3333333095802695, 2.000000017707398};


__device__ __forceinline__ float sa_expf(float x) {
  const bool nan = x != x;
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
  const int ki = nan ? 0 : (int)k;
  const float res = ldexpf(p, ki);
  return nan ? x : res;
}

// sa_expf for callers whose result is NaN whenever x is NaN anyway (x / (1 +
// exp(..x..)) forms): the same value for every non-NaN x, without the NaN
// bookkeeping, and the clamp is one v_med3.
__device__ __forceinline__ float sa_expf_nn(float x) {
  x = __builtin_amdgcn_fmed3f(x, -104.0f, 89.0f);
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

__device__ __forceinline__ float sa_logf(float x) {
  const bool tiny = x < 1.17549435e-38f;
  const float xs = tiny ? x * 8388608.0f : x;
  const uint32_t ix = __float_as_uint(xs) - 0x3f3504f3u;
  const int e = ((int32_t)ix >> 23) + (tiny ? -23 : 0);
  const float f = __uint_as_float((ix & 0x007fffffu) + 0x3f3504f3u) - 1.0f;
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
  float r = fmaf(ef, 0.693145751953125f, fmaf(ef, 1.42860677e-06f, y));
  // special cases: NaN and negative -> NaN, 0 -> -inf, +inf -> +inf
  r = (x == __builtin_inff()) ? x : r;
  r = (x == 0.0f) ? -__builtin_inff() : r;
  r = (x < 0.0f || x != x) ? __builtin_nanf("") : r;
  return r;
}

// sa_logf for finite normal x > 0 (callers whose NaN inputs turn the result
// NaN elsewhere): the same value there, without the special-case selects.
__device__ __forceinline__ float sa_logf_normal(float x) {
  const uint32_t ix = __float_as_uint(x) - 0x3f3504f3u;
  const int e = (int32_t)ix >> 23;
  const float f = __uint_as_float((ix & 0x007fffffu) + 0x3f3504f3u) - 1.0f;
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

// erf in binary32, <= 0.978 ulp over every input (1.5 % of results not
// correctly rounded).  Three ranges of |x|:
//   [0, 0.921875):     x + x P(x^2), P of degree 6 (relative error 2^-31);
//   [0.921875, 2.25):  1 - M(|x| - 1.5859375), M ~ erfc of degree 9;
//   [2.25, 3.9375):    1 - T(|x| - 3.09375),   T ~ erfc of degree 9
//                      (absolute errors 2^-27); +-1 beyond.
// The subtractions |x| - c are exact (Sterbenz).  A branch per range: a
// wavefront pays for every range one of its lanes falls in, and for N(0, 1)
// data only about one wavefront-element in eleven reaches the tail range.
// sa_erff without the NaN select, for callers whose result is NaN for a NaN
// x anyway (gelu's (x/2)(1 + erf)): the same value for every other x.
__device__ __forceinline__ float sa_erff_nn(float x) {
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
  return r;
}

__device__ __forceinline__ float sa_erff(float x) { return (x != x) ? x : sa_erff_nn(x); }

// expm1: sa_expf's reduction and polynomial (r + r^2 P(r) is e^r - 1), then
// 2^k (e^r - 1) + (2^k - 1), or 2^k e^r - 1 from k = 25 on.
__device__ __forceinline__ float sa_expm1f(float x) {
  const bool nan = x != x;
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
  const int ki = nan ? 0 : (int)k;
  const float big = ldexpf(q + 1.0f, ki) - 1.0f;
  const float small = ldexpf(q, ki) + (ldexpf(1.0f, ki) - 1.0f);
  const float res = ki >= 25 ? big : small;
  return nan ? x : res;
}

// log1p: log(u) + (z - (u - 1)) / u with u = 1 + z rounded, for |z| <= 1;
// log(u) beyond.  z = -1 gives -inf, z < -1 NaN.
__device__ __forceinline__ float sa_log1pf(float z) {
  const float u = 1.0f + z;
  const float c = (fabsf(z) <= 1.0f) ? z - (u - 1.0f) : 0.0f;
  const float r = sa_logf(u) + c / u;
  return (u == 0.0f) ? -__builtin_inff() : r;
}

// Normal CDF pieces for gelu 'none': with t = |x| / sqrt(2) (clamped to
// 3.925), E = erfc(t) = exp(L(t)), L ~ log(erfc) fitted on [0, 3.925]
// (degree 11).  Then gelu(x) = x - (x/2) E for x >= 0 and (x/2) E for x < 0
// -- the same function as x (1 + erf(x / sqrt 2)) / 2 without the
// cancellation of 1 + erf for x << 0 -- and x or -0 once t > 3.925.
__device__ __forceinline__ float sa_erfc_core(float x) {
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
  return sa_expf_nn(l);  // l in [-17.5, 0]
}
__device__ __forceinline__ float sa_gelu_none(float x) {
  const float t = fabsf(x) * 0.70710678118654752f;
  const float e = sa_erfc_core(x);
  const float hx = 0.5f * x;
  float g = (x >= 0.0f) ? fmaf(-hx, e, x) : hx * e;  // a NaN x stays NaN
  g = (t > 3.925f) ? ((x >= 0.0f) ? x : x * 0.0f) : g;
  return g;
}
// Phi(x) = P(N(0, 1) <= x) through the same E: 1 - E/2 or E/2.
__device__ __forceinline__ float sa_phif(float x) {
  const float t = fabsf(x) * 0.70710678118654752f;
  const float e = sa_erfc_core(x);
  float p = (x >= 0.0f) ? fmaf(-0.5f, e, 1.0f) : 0.5f * e;
  p = (t > 3.925f) ? ((x >= 0.0f) ? 1.0f : 0.0f) : p;
  return (x != x) ? x : p;
}

// tanh's binary64 core, for |x|: with a = min(|x|, 9.5) (tanh(9.5) rounds to
// 1 in binary32), 2a = k ln2 + 2s, |s| <= ln2/4, k from the 1.5 * 2^52
// shifter (the low word of the sum is k); e^{2s} - 1 = s (2 + s Q(s)), Q of
// degree 5 (relative error 2^-32.0); m = e^{2a} - 1 = 2^k (e^{2s} - 1) +
// (2^k - 1), 2^k built from its exponent field, which keeps m's relative
// accuracy as a -> 0; h = m + 2; tanh(a) = m / h.  The callers give the
// result x's sign, so tanh(-x) = -tanh(x) exactly.  A NaN x yields a number
// here.
__device__ __forceinline__ void sa_tanh_mh(float x, double& m, double& h) {
  const float a = fminf(fabsf(x), 9.5f);
  const double d = (double)a;
  const double kb = fma(d, 2.8853900817779268, 6755399441055744.0);  // 2 / ln2, 1.5 * 2^52
  const double k = kb - 6755399441055744.0;
  const double s = fma(-k, 0.34657359027997264, d);  // a - k ln2 / 2
  double q = kTanhQ[0];
#pragma unroll
  for (int i = 1; i < 6; ++i) q = fma(q, s, kTanhQ[i]);
  const double e = s * fma(s, q, 2.0);  // e^{2s} - 1
  const double p2 = __hiloint2double((__double2loint(kb) + 1023) << 20, 0);
  m = fma(p2, e, p2 - 1.0);  // e^{2a} - 1
  h = m + 2.0;
}
// m / h to within 2^-48.5 (relative): the hardware reciprocal seed
// (v_rcp_f64, relative error below 2^-24 on this range) and one Newton step
// give y = (1 / h)(1 + e), |e| <= 2^-48.7, and m * y rounds once more.
__device__ __forceinline__ double sa_tanh_quot_fast(double m, double h) {
  double y = __builtin_amdgcn_rcp(h);
  y = fma(y, fma(-h, y, 1.0), y);
  return m * y;
}
// m / h correctly rounded to binary64: the quotient q0 of sa_tanh_quot_fast
// and one correction q0 + r y with the residual r = m - h q0 (one fma, exact
// but for a rounding 2^-53 relative to r).  Before its final rounding the
// corrected value is m / h within 2^-97 (relative), so it rounds to the
// binary64 quotient unless m / h lies that close to a binary64 rounding
// midpoint, where a quotient of two binary64 numbers can come within 2^-107
// but, over uniformly placed values, with probability 2^-44 per element;
// the binary32 result then changes only if that binary64 value is also a
// binary32 rounding boundary.  Any IEEE binary64 division m / h is therefore
// the reproducible restatement of this value.
__device__ __forceinline__ double sa_tanh_quot(double m, double h) {
  double y = __builtin_amdgcn_rcp(h);
  y = fma(y, fma(-h, y, 1.0), y);
  const double q0 = m * y;
  const double r = fma(-h, q0, m);
  return fma(r, y, q0);
}
__device__ __forceinline__ double sa_tanh_core(float x) {
  double m, h;
  sa_tanh_mh(x, m, h);
  return sa_tanh_quot(m, h);
}
// The core with the quotient of sa_tanh_quot_fast: the same binary32 value
// as sa_tanh_core except where m / h lies within 2^-48.5 (relative) of a
// binary32 rounding boundary (about one element in 2^24), where it may be the
// other neighbour.  Two binary64 fma fewer per element; gelu('tanh') forward
// uses it.
__device__ __forceinline__ float sa_tanhf_fast_nn(float x) {
  double m, h;
  sa_tanh_mh(x, m, h);
  return copysignf((float)sa_tanh_quot_fast(m, h), x);
}
__device__ __forceinline__ float sa_tanhf(float x) {
  const float y = copysignf((float)sa_tanh_core(x), x);
  return (x != x) ? x : y;
}

}  // namespace sa
