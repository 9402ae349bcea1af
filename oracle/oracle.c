/*
 * TEST INFRASTRUCTURE ONLY -- the CPU oracle of the elementwise + loss path.
 *
 * A plain-C restatement of the arithmetic the reference runs on its device for
 * each op, written from the reference sources cited per function.  Only
 * tests/, bench.py's cpu_baseline leg and __graft_entry__.smoke() may load it,
 * and only as the checker; the shipped library never links or calls it.
 *
 * Conventions.
 *  - Arrays are flat and contiguous: broadcasting and dtype plumbing are done
 *    by the numpy wrapper (oracle/__init__.py) before the call.
 *  - bfloat16 is carried as uint16 bit patterns; conversions are round to
 *    nearest even with NaN -> 0x7FC0, the rule of c10::BFloat16.
 *  - "opmath" is float32 for f32/bf16/f16 storage, as in the reference's
 *    at::opmath_type.
 *  - Elementwise formulas keep the operation order of the reference functor so
 *    the float32 result is bit-identical to an IEEE device that evaluates the
 *    same sequence.  Row and full reductions accumulate in double here, so the
 *    device (which accumulates in float32 in a different order) is compared
 *    with a tolerance, not bit for bit.
 *
 * Build: oracle/Makefile (gcc -O2 -march=x86-64-v3 -ffp-contract=off).
 * Parity of every function is pinned by tests/test_oracle_*.py against the
 * upstream aten CPU kernels (torch 2.10.0, the kernels the reference's
 * operator library is built from), committed golden vectors, closed forms and
 * invariants.
 */
#include "oracle_math.h"

#include <stddef.h>
#include <stdint.h>
#include <stdlib.h>

/* ---------------------------------------------------------------- casts -- */

/* c10/util/BFloat16.h round_to_nearest_even (NaN -> 0x7FC0). */
static inline uint16_t bf16_from_f32(float f) {
  if (isnan(f)) return 0x7FC0u;
  const uint32_t u = or_as_u32(f);
  return (uint16_t)((u + (((u >> 16) & 1u) + 0x7FFFu)) >> 16);
}
static inline float bf16_to_f32(uint16_t h) { return or_as_float((uint32_t)h << 16); }

void or_f32_to_bf16(const float* in, uint16_t* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = bf16_from_f32(in[i]);
}
void or_bf16_to_f32(const uint16_t* in, float* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = bf16_to_f32(in[i]);
}
void or_f64_to_bf16(const double* in, uint16_t* out, int64_t n) {
  /* Direct RNE from double (used for exact-math references of bf16 results). */
  for (int64_t i = 0; i < n; ++i) {
    const double d = in[i];
    if (isnan(d)) { out[i] = 0x7FC0u; continue; }
    const float f = (float)d; /* may round; fix up a double-rounding tie below */
    uint16_t h = bf16_from_f32(f);
    const double lo = (double)bf16_to_f32(h);
    /* choose the nearer of h and its neighbour towards d */
    const uint16_t h2 = (uint16_t)(d > lo ? h + ((h & 0x8000u) ? -1 : 1)
                                          : h + ((h & 0x8000u) ? 1 : -1));
    if (d != lo && !isinf(lo)) {
      const double alt = (double)bf16_to_f32(h2);
      if (fabs(alt - d) < fabs(lo - d)) h = h2;
    }
    out[i] = h;
  }
}

/* ------------------------------------------------------------ binary ops -- */

enum { OR_ADD = 0, OR_MUL = 1, OR_DIV = 2, OR_DIV_TRUNC = 3, OR_DIV_FLOOR = 4, OR_MAX = 5, OR_MIN = 6 };

/* maximum / minimum (upstream MaxMinElementwiseKernel.cu): a NaN operand is
 * the result. */
static inline float max_nan_f32(float a, float b) { return isnan(a) ? a : (isnan(b) ? b : (a > b ? a : b)); }
static inline float min_nan_f32(float a, float b) { return isnan(a) ? a : (isnan(b) ? b : (a < b ? a : b)); }

/* c10::div_floor_floating (c10/util/generic_math.h), the Python-style floor
 * division that BinaryDivFloorKernel.cu:22-82 applies to floating types. */
static inline float div_floor_f32(float a, float b) {
  if (b == 0.0f) return a / b;
  float mod = fmodf(a, b);
  float div = (a - mod) / b;
  if (mod != 0.0f && ((b < 0.0f) != (mod < 0.0f))) div -= 1.0f;
  float floordiv;
  if (div != 0.0f) {
    floordiv = floorf(div);
    if (div - floordiv > 0.5f) floordiv += 1.0f;
  } else {
    floordiv = copysignf(0.0f, a / b);
  }
  return floordiv;
}
static inline double div_floor_f64(double a, double b) {
  if (b == 0.0) return a / b;
  double mod = fmod(a, b);
  double div = (a - mod) / b;
  if (mod != 0.0 && ((b < 0.0) != (mod < 0.0))) div -= 1.0;
  double floordiv;
  if (div != 0.0) {
    floordiv = floor(div);
    if (div - floordiv > 0.5) floordiv += 1.0;
  } else {
    floordiv = copysign(0.0, a / b);
  }
  return floordiv;
}

/* add: ufunc::add `self + alpha * other` in opmath (UfuncCUDA_add.cu:13-16),
 *      evaluated as one fused multiply-add (the contraction both the CUDA
 *      compiler and the CPU vectorised kernel apply);
 * mul: MulFunctor (BinaryInternal.h:17-22);
 * div: DivFunctor `a / b` (BinaryInternal.h:10-15), true IEEE division;
 * div trunc / floor: BinaryDivTruncKernel.cu:22-55 / BinaryDivFloorKernel.cu:22-82. */
void or_binary_f32(int op, const float* a, const float* b, float* out, int64_t n, float alpha) {
  for (int64_t i = 0; i < n; ++i) {
    const float x = a[i], y = b[i];
    float r;
    switch (op) {
      case OR_ADD: r = fmaf(alpha, y, x); break;
      case OR_MUL: r = x * y; break;
      case OR_DIV: r = x / y; break;
      case OR_DIV_TRUNC: r = truncf(x / y); break;
      case OR_MAX: r = max_nan_f32(x, y); break;
      case OR_MIN: r = min_nan_f32(x, y); break;
      default: r = div_floor_f32(x, y); break;
    }
    out[i] = r;
  }
}
void or_binary_f64(int op, const double* a, const double* b, double* out, int64_t n, double alpha) {
  for (int64_t i = 0; i < n; ++i) {
    const double x = a[i], y = b[i];
    double r;
    switch (op) {
      case OR_ADD: r = fma(alpha, y, x); break;
      case OR_MUL: r = x * y; break;
      case OR_DIV: r = x / y; break;
      case OR_DIV_TRUNC: r = trunc(x / y); break;
      default: r = div_floor_f64(x, y); break;
    }
    out[i] = r;
  }
}

/* ---------------------------------------------------- ternary pointwise -- */

enum { OR_ADDCMUL = 0, OR_ADDCDIV = 1, OR_LERP = 2 };

/* addcmul / addcdiv: self + value * (t1 op t2) with the product-sum as one
 * fma (upstream CUDA PointwiseOpsKernel.cu / ForeachPointwiseOp.cu as the
 * CUDA compiler contracts it); lerp: upstream Lerp.h,
 * |w| < 0.5 ? self + w (end - self) : end - (end - self)(1 - w), each
 * product-sum one fma.  c is t2 (addc*) or the weight (lerp). */
void or_ternary_f32(int op, const float* a, const float* b, const float* c, float* out, int64_t n, float value) {
  for (int64_t i = 0; i < n; ++i) {
    const float x = a[i], y = b[i], z = c[i];
    float r;
    switch (op) {
      case OR_ADDCMUL: r = fmaf(value, y * z, x); break;
      case OR_ADDCDIV: r = fmaf(value, y / z, x); break;
      default: {
        const float d = y - x;
        r = fabsf(z) < 0.5f ? fmaf(z, d, x) : fmaf(-d, 1.0f - z, y);
        break;
      }
    }
    out[i] = r;
  }
}


/* -------------------------------------------------------- activations -- */

enum {
  OR_GELU = 0, OR_GELU_TANH = 1, OR_SILU = 2, OR_SIGMOID = 3, OR_TANH = 4,
  OR_EXP = 5, OR_LOG = 6, OR_ERF = 7, OR_RELU = 8, OR_NEG = 9, OR_RECIPROCAL = 10, OR_ABS = 11,
  OR_SQRT = 12, OR_EXPM1 = 13, OR_LOG1P = 14,
  /* the opt-in cancellation-free gelu forms (same codes as the C ABI) */
  OR_GELU_LOGERFC = 22, OR_GELU_TANH_LOGISTIC = 23,
  /* oracle only: gelu('tanh') with or_tanhf_fast_alt's neighbour (the other
   * value the device's forward may return) */
  OR_GELU_TANH_FAST_ALT = 100
};

#define OR_SQRT1_2 0.70710678118654752440f
#define OR_GELU_BETA_NONE 0.3989422804014327f /* M_2_SQRTPI * M_SQRT1_2 * 0.5 */
#define OR_GELU_BETA_TANH 0.7978845608028654f /* M_SQRT2 * M_2_SQRTPI * 0.5  */
#define OR_GELU_KAPPA 0.044715f

/* Forward formulas (all in float32 opmath), in the reference's operation
 * order (upstream GeluKernel.cu / CPU Gelu.h:34-41, 61-65):
 *  gelu 'none': (x*0.5)*(1+erf(x*M_SQRT1_2))          NF:5216, CPU Gelu.h:61-65
 *  gelu 'tanh': (0.5*x)*(1+tanh(b*(x+k*x^3))), x^3 = (x*x)*x and x + k*x^3
 *               one fused multiply-add (the contraction the reference's
 *               compilers apply)                       NF:5216, CPU Gelu.h:34-41
 *  silu:        x / (1 + exp(-x))                      NF:5374
 *  sigmoid:     1 / (1 + exp(-x))                      NF:5441
 *  tanh, exp, log, erf, expm1, log1p: the primitives of oracle_math.h;
 *  reciprocal, abs, sqrt: IEEE 1/x, |x| and correctly rounded sqrt.
 * Opt-in forms (not the reference's arithmetic; they avoid the cancellation
 * of 1 + erf and 1 + tanh for x << 0):
 *  GELU_LOGERFC:        x - (x/2) erfc(|x|/sqrt2) (x >= 0), (x/2) erfc(|x|/sqrt2)
 *                       (x < 0), erfc through log erfc (or_gelu_none)
 *  GELU_TANH_LOGISTIC:  x / (1 + exp(-2*b*(x+k*x^3))) (the identity
 *                       0.5*(1+tanh(u)) = 1/(1+exp(-2u))) */
static inline float gelu_tanh_inner(float x) {
  const float x3 = (x * x) * x;
  return OR_GELU_BETA_TANH * fmaf(OR_GELU_KAPPA, x3, x);
}
static inline float act_fwd(int op, float x) {
  switch (op) {
    case OR_GELU: return (x * 0.5f) * (1.0f + or_erff_nn(x * OR_SQRT1_2));
    case OR_GELU_TANH: return (0.5f * x) * (1.0f + or_tanhf(gelu_tanh_inner(x)));
    case OR_GELU_TANH_FAST_ALT: return (0.5f * x) * (1.0f + or_tanhf_fast_alt(gelu_tanh_inner(x)));
    case OR_GELU_LOGERFC: return or_gelu_none(x);
    case OR_GELU_TANH_LOGISTIC: {
      const float x3 = (x * x) * x;
      const float inner = (-2.0f * OR_GELU_BETA_TANH) * fmaf(OR_GELU_KAPPA, x3, x);
      return x / (1.0f + or_expf(inner));
    }
    case OR_SILU: return x / (1.0f + or_expf(-x));
    case OR_SIGMOID: return 1.0f / (1.0f + or_expf(-x));
    case OR_TANH: return or_tanhf(x);
    case OR_EXP: return or_expf(x);
    case OR_LOG: return or_logf(x);
    case OR_ERF: return or_erff(x);
    case OR_RELU: return (x != x) ? x : (x > 0.0f ? x : 0.0f);
    case OR_RECIPROCAL: return 1.0f / x;
    case OR_ABS: return fabsf(x);
    case OR_SQRT: return sqrtf(x);
    case OR_EXPM1: return or_expm1f(x);
    case OR_LOG1P: return or_log1pf(x);
    default: return -x;
  }
}

/* Backward formulas (upstream aten activation backward functors, float32):
 *  gelu 'none': dy*(cdf + x*pdf), cdf = 0.5*(1+erf(x*M_SQRT1_2)),
 *               pdf = exp(-0.5*x*x) * (M_2_SQRTPI*M_SQRT1_2*0.5)      NF:5245
 *               (GELU_LOGERFC: cdf = Phi(x) through the same erfc as its
 *               forward, or_phif)
 *  gelu 'tanh': dy*(0.5*(1+t) + 0.5*x*(1-t*t)*b*(1+3k*x^2)),
 *               t = tanh(b*(x+k*x^3))                                NF:5245
 *  silu:        s = 1/(1+exp(-x)); dy*s*(1+x*(1-s))                  NF:5383
 *  sigmoid:     dy*(1-y)*y        (input is the forward output y)    NF:13229
 *  tanh:        dy*(1-y*y)        (input is the forward output y) */
static inline float act_bwd(int op, float dy, float x) {
  switch (op) {
    case OR_GELU:
    case OR_GELU_LOGERFC: {
      const float cdf = (op == OR_GELU) ? 0.5f * (1.0f + or_erff_nn(x * OR_SQRT1_2)) : or_phif(x);
      const float pdf = or_expf((-0.5f * x) * x) * OR_GELU_BETA_NONE;
      return dy * fmaf(x, pdf, cdf);
    }
    case OR_GELU_TANH:
    case OR_GELU_TANH_LOGISTIC: {
      const float x2 = x * x;
      const float x3 = x2 * x;
      const float inner = OR_GELU_BETA_TANH * fmaf(OR_GELU_KAPPA, x3, x);
      const float t = or_tanhf(inner);
      const float left = 0.5f * x;
      const float right = 1.0f + t;
      const float left_d = 0.5f * right;
      const float right_d = fmaf(-t, t, 1.0f);
      const float inner_d = OR_GELU_BETA_TANH * fmaf(3.0f * OR_GELU_KAPPA, x2, 1.0f);
      return dy * fmaf(left * right_d, inner_d, left_d);
    }
    case OR_SILU: {
      const float s = 1.0f / (1.0f + or_expf(-x));
      return (dy * s) * fmaf(x, 1.0f - s, 1.0f);
    }
    case OR_SIGMOID: return (dy * (1.0f - x)) * x;
    case OR_TANH: return dy * fmaf(-x, x, 1.0f);
    default: return dy;
  }
}

void or_unary_f32(int op, const float* x, float* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = act_fwd(op, x[i]);
}
void or_unary_backward_f32(int op, const float* dy, const float* x, float* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = act_bwd(op, dy[i], x[i]);
}

/* --------------------------------------- parameterised activations -- */

enum {
  OR_ACT_LEAKY_RELU = 0, OR_ACT_HARDTANH = 1, OR_ACT_ELU = 2, OR_ACT_SOFTPLUS = 3, OR_ACT_HARDSWISH = 4,
  OR_ACT_HARDSIGMOID = 5, OR_ACT_MISH = 6, OR_ACT_LOG_SIGMOID = 7, OR_ACT_THRESHOLD = 8
};

/* std::max / std::min as the device code of upstream's kernels evaluates
 * them: (a < b) ? b : a and (b < a) ? b : a (a NaN first operand passes). */
static inline float max_lt(float a, float b) { return (a < b) ? b : a; }
static inline float min_lt(float a, float b) { return (b < a) ? b : a; }

/* Forward formulas of upstream's CUDA activation kernels (ActivationLeakyReluKernel.cu,
 * ActivationEluKernel.cu, ActivationSoftplusKernel.cu, ActivationHardswishKernel.cu,
 * ActivationHardsigmoidKernel.cu, ActivationMishKernel.cu, ActivationLogSigmoidKernel.cu,
 * ActivationThresholdKernel.cu), float32 opmath, parameters rounded to float:
 *  leaky_relu  x > 0 ? x : x*p0                                     NF:12226
 *  elu         x > 0 ? x*p1 : expm1(x*p2) * (p0*p1)  (alpha, scale, input_scale)  NF:12065
 *  softplus    x*p0 > p1 ? x : log1p(exp(x*p0)) / p0  (beta, threshold)  NF:12327
 *  hardswish   x * min(max(x+3, 0), 6) * (1/6)                      NF:12199
 *  hardsigmoid min(max(x+3, 0), 6) * (1/6)                          NF:12135
 *  mish        x * tanh(log1p(exp(x)))                              NF:5400
 *  log_sigmoid min(0, x) - log1p(exp(-|x|))                         NF:12268
 *  threshold   x <= p0 ? p1 : x                                     NF:6231
 * (hardtanh's forward is clamp.) */
static inline float act_p_fwd(int act, float x, float p0, float p1, float p2) {
  switch (act) {
    case OR_ACT_LEAKY_RELU: return x > 0.0f ? x : x * p0;
    case OR_ACT_ELU: return x > 0.0f ? x * p1 : or_expm1f(x * p2) * (p0 * p1);
    case OR_ACT_SOFTPLUS: return (x * p0) > p1 ? x : or_log1pf(or_expf(x * p0)) / p0;
    case OR_ACT_HARDSWISH: return (x * min_lt(max_lt(x + 3.0f, 0.0f), 6.0f)) * (1.0f / 6.0f);
    case OR_ACT_HARDSIGMOID: return min_lt(max_lt(x + 3.0f, 0.0f), 6.0f) * (1.0f / 6.0f);
    case OR_ACT_MISH: return x * or_tanhf(or_log1pf(or_expf(x)));
    case OR_ACT_LOG_SIGMOID: return min_lt(0.0f, x) - or_log1pf(or_expf(-fabsf(x)));
    case OR_ACT_THRESHOLD: return x <= p0 ? p1 : x;
    default: return x;
  }
}

/* Backward formulas (the same files' backward functors; g the incoming
 * gradient, x the forward input -- the forward output for elu with flag set);
 * `a + b*c` forms are one fma, as upstream's compiler contracts them:
 *  leaky_relu  x > 0 ? g : g*p0                                     NF:12241
 *  hardtanh    x <= p0 || x >= p1 ? 0 : g  (min, max)               NF:12180
 *  elu         result form: x <= 0 ? g*p2*(x + p0*p1) : g*p1;
 *              input form:  x <= 0 ? g*p2*(p0*p1)*exp(x*p2) : g*p1  NF:12078
 *  softplus    z = exp(x*p0); x*p0 > p1 ? g : g*z/(z+1)             NF:12341
 *  hardswish   x < -3 ? 0 : x <= 3 ? g*(x/3 + 0.5) : g              NF:12211
 *  hardsigmoid -3 < x < 3 ? g/6 : 0                                 NF:12155
 *  mish        s = 1/(1+exp(-x)), t = tanh(log1p(exp(x))); g*(t + x*s*(1 - t*t))  NF:5417
 *  log_sigmoid z = exp(-|x|); g*(d - sg * z/(1+z)), d = x<0, sg = x<0 ? 1 : -1  NF:12283
 *  threshold   x <= p0 ? 0 : g                                      NF:6261 */
static inline float act_p_bwd(int act, float g, float x, float p0, float p1, float p2, int flag) {
  switch (act) {
    case OR_ACT_LEAKY_RELU: return x > 0.0f ? g : g * p0;
    case OR_ACT_HARDTANH: return (x <= p0 || x >= p1) ? 0.0f : g;
    case OR_ACT_ELU: {
      const float negcoef = p0 * p1;
      if (flag) return x <= 0.0f ? (g * p2) * (x + negcoef) : g * p1;
      return x <= 0.0f ? ((g * p2) * negcoef) * or_expf(x * p2) : g * p1;
    }
    case OR_ACT_SOFTPLUS: {
      const float z = or_expf(x * p0);
      return (x * p0) > p1 ? g : (g * z) / (z + 1.0f);
    }
    case OR_ACT_HARDSWISH: return x < -3.0f ? 0.0f : (x <= 3.0f ? g * ((x / 3.0f) + 0.5f) : g);
    case OR_ACT_HARDSIGMOID: return (x > -3.0f && x < 3.0f) ? g * (1.0f / 6.0f) : 0.0f;
    case OR_ACT_MISH: {
      const float sg = 1.0f / (1.0f + or_expf(-x));
      const float t = or_tanhf(or_log1pf(or_expf(x)));
      return g * fmaf(x * sg, fmaf(-t, t, 1.0f), t);
    }
    case OR_ACT_LOG_SIGMOID: {
      const int neg = x < 0.0f;
      const float z = or_expf(-fabsf(x));
      return g * fmaf(neg ? -1.0f : 1.0f, z / (1.0f + z), neg ? 1.0f : 0.0f);
    }
    case OR_ACT_THRESHOLD: return x <= p0 ? 0.0f : g;
    default: return g;
  }
}

void or_activation_f32(int act, const float* x, float* out, int64_t n, float p0, float p1, float p2) {
  for (int64_t i = 0; i < n; ++i) out[i] = act_p_fwd(act, x[i], p0, p1, p2);
}
void or_activation_backward_f32(int act, const float* g, const float* x, float* out, int64_t n, float p0, float p1,
                                float p2, int flag) {
  for (int64_t i = 0; i < n; ++i) out[i] = act_p_bwd(act, g[i], x[i], p0, p1, p2, flag);
}

/* ---------------------------------------------------------- log_softmax -- */

/* _log_softmax over the last dim (NF:3752; upstream SoftMax.cu epilogue
 * `input - max - log(sum(exp(input - max)))`).  max is exact; the sum is
 * accumulated in double, log(sum) rounded to float, and the output formed in
 * float as (x - max) - logsum, the order of the upstream epilogue. */
void or_log_softmax_fwd(const float* x, float* out, int64_t rows, int64_t cols) {
  for (int64_t r = 0; r < rows; ++r) {
    const float* xr = x + r * cols;
    float* o = out + r * cols;
    float mx = -INFINITY;
    for (int64_t c = 0; c < cols; ++c) mx = (xr[c] > mx || isnan(xr[c])) ? xr[c] : mx;
    double s = 0.0;
    for (int64_t c = 0; c < cols; ++c) s += exp((double)xr[c] - (double)mx);
    const float logsum = (float)log(s);
    for (int64_t c = 0; c < cols; ++c) o[c] = (xr[c] - mx) - logsum;
  }
}

/* _log_softmax_backward_data (NF:3763): gI = gO - exp(out) * sum(gO) per row;
 * sum in double, rounded to float; exp(out) exact in double then rounded. */
void or_log_softmax_bwd(const float* g, const float* y, float* gin, int64_t rows, int64_t cols) {
  for (int64_t r = 0; r < rows; ++r) {
    const float* gr = g + r * cols;
    const float* yr = y + r * cols;
    double s = 0.0;
    for (int64_t c = 0; c < cols; ++c) s += (double)gr[c];
    const float sf = (float)s;
    for (int64_t c = 0; c < cols; ++c) gin[r * cols + c] = gr[c] - (float)exp((double)yr[c]) * sf;
  }
}

/* _softmax (NF:5690; upstream SoftMax.cu epilogue exp(x - max) / sum): the
 * row max as float, the sum of exp(x - max) in double, each output
 * exp(x - max) / sum in double rounded to float. */
void or_softmax_fwd(const float* x, float* out, int64_t rows, int64_t cols) {
  for (int64_t r = 0; r < rows; ++r) {
    const float* xr = x + r * cols;
    float* o = out + r * cols;
    float mx = -INFINITY;
    for (int64_t c = 0; c < cols; ++c) mx = (xr[c] > mx || isnan(xr[c])) ? xr[c] : mx;
    double s = 0.0;
    for (int64_t c = 0; c < cols; ++c) s += exp((double)xr[c] - (double)mx);
    for (int64_t c = 0; c < cols; ++c) o[c] = (float)(exp((double)xr[c] - (double)mx) / s);
  }
}

/* _softmax_backward_data (NF:5704; upstream SoftMaxBackwardEpilogue):
 * gI = out * (gO - sum(gO * out)) per row, the sum in double rounded to float. */
void or_softmax_bwd(const float* g, const float* y, float* gin, int64_t rows, int64_t cols) {
  for (int64_t r = 0; r < rows; ++r) {
    const float* gr = g + r * cols;
    const float* yr = y + r * cols;
    double s = 0.0;
    for (int64_t c = 0; c < cols; ++c) s += (double)gr[c] * (double)yr[c];
    const float sf = (float)s;
    for (int64_t c = 0; c < cols; ++c) gin[r * cols + c] = yr[c] * (gr[c] - sf);
  }
}

/* ------------------------------------------------------------- nll_loss -- */

/* nll_loss_forward (NF:11928; reference semantics CrossEntropyLossKernel.cu:71-119
 * for ignore handling): rows whose target == ignore_index contribute nothing
 * and are not counted.  reduction 0 none / 1 mean / 2 sum.  For mean the
 * result is -sum/total_weight (NaN when every row is ignored).  weight may be
 * NULL.  Accumulation in double.  Returns 0, or -1 on an out-of-range target. */
int or_nll_loss_fwd(const float* logp, const int64_t* target, const float* weight,
                    int64_t n, int64_t c, int reduction, int64_t ignore_index,
                    float* out, float* total_weight) {
  double acc = 0.0, tw = 0.0;
  for (int64_t i = 0; i < n; ++i) {
    const int64_t t = target[i];
    if (t == ignore_index) { if (reduction == 0) out[i] = 0.0f; continue; }
    if (t < 0 || t >= c) return -1;
    const float w = weight ? weight[t] : 1.0f;
    const float v = -w * logp[i * c + t];
    if (reduction == 0) out[i] = v;
    acc += (double)v;
    tw += (double)w;
  }
  if (reduction == 0) { *total_weight = 0.0f; return 0; }
  *total_weight = (float)tw;
  out[0] = reduction == 1 ? (float)(acc / tw) : (float)acc;
  return 0;
}

/* nll_loss_backward (NF:11940): grad_input is zero except
 * grad_input[i, t_i] = -w[t_i] * g_i (none) or -w[t_i] * g / total_weight
 * (mean) or -w[t_i] * g (sum); ignored rows stay zero.  total_weight is the
 * stored forward value, so a bf16 total_weight enters rounded, as upstream.
 * bf16 != 0 applies the storage-type rounding of a bfloat16 run. */
int or_nll_loss_bwd(const float* grad_out, const int64_t* target, const float* weight,
                    int64_t n, int64_t c, int reduction, int64_t ignore_index,
                    float total_weight, int bf16, float* grad_in) {
  for (int64_t i = 0; i < n * c; ++i) grad_in[i] = 0.0f;
  for (int64_t i = 0; i < n; ++i) {
    const int64_t t = target[i];
    if (t == ignore_index) continue;
    if (t < 0 || t >= c) return -1;
    const float w = weight ? weight[t] : 1.0f;
    float g = reduction == 0 ? grad_out[i] : grad_out[0];
    if (reduction == 1) g = g / total_weight;
    /* upstream forms -(g/total_weight) in the storage type (scalar_t), so a
     * bf16 run rounds it before the weight multiply */
    if (bf16) g = bf16_to_f32(bf16_from_f32(g));
    grad_in[i * c + t] = weight ? w * -g : -g;
  }
  return 0;
}

/* ------------------------------------------------- fused cross-entropy -- */

/* Cross-entropy over logits [n, c] with int64 targets, in double: the
 * reference's fast-path row loss lse_i - x[i, t_i], lse_i = max + log(sum
 * exp(x - max)) (CrossEntropyLossKernel.cu:71-119), ignore_index rows
 * contributing 0 and not counted, mean = sum / count (NaN for count 0,
 * :191-193).  reduction: 0 none (loss[n]), 1 mean, 2 sum (loss[0]).  lse[n]
 * is written (0 for ignored rows) and *count receives the kept-row count.
 * Returns -1 for an out-of-range target. */
int or_ce_fwd(const double* x, const int64_t* target, int64_t n, int64_t c, int64_t ignore_index,
              int reduction, double* loss, double* lse, double* count) {
  double sum = 0.0, cnt = 0.0;
  for (int64_t i = 0; i < n; ++i) {
    const int64_t t = target[i];
    const double* r = x + i * c;
    if (t == ignore_index) {
      lse[i] = 0.0;
      if (reduction == 0) loss[i] = 0.0;
      continue;
    }
    if (t < 0 || t >= c) return -1;
    double m = -INFINITY;
    for (int64_t j = 0; j < c; ++j) m = r[j] > m ? r[j] : m;
    double s = 0.0;
    for (int64_t j = 0; j < c; ++j) s += exp(r[j] - m);
    const double l = m + log(s);
    lse[i] = l;
    if (reduction == 0) loss[i] = l - r[t];
    sum += l - r[t];
    cnt += 1.0;
  }
  if (reduction == 1) loss[0] = sum / cnt;
  else if (reduction == 2) loss[0] = sum;
  *count = cnt;
  return 0;
}

/* Its gradient: (exp(x - lse_i) - [j == t_i]) * g_i, g_i = g[i] (none),
 * g / count (mean), g (sum); ignored rows 0.  This is what the reference's
 * backward composition nll_loss_backward + _log_softmax_backward_data
 * computes (CrossEntropyLoss.cpp:94-135): grad_lp = -g_i at t_i, and
 * grad_x = grad_lp - softmax * sum(grad_lp). */
void or_ce_bwd(const double* g, const double* x, const int64_t* target, const double* lse, double count,
               int64_t n, int64_t c, int64_t ignore_index, int reduction, double* gx) {
  for (int64_t i = 0; i < n; ++i) {
    const int64_t t = target[i];
    double* o = gx + i * c;
    if (t == ignore_index || t < 0 || t >= c) {
      for (int64_t j = 0; j < c; ++j) o[j] = 0.0;
      continue;
    }
    const double gi = reduction == 0 ? g[i] : (reduction == 1 ? g[0] / count : g[0]);
    const double* r = x + i * c;
    for (int64_t j = 0; j < c; ++j) o[j] = (exp(r[j] - lse[i]) - (j == t ? 1.0 : 0.0)) * gi;
  }
}

/* Cross-entropy with probability targets, in float64 (t: [n, c] class
 * probabilities): loss_i = sum_j t_ij (lse_i - x_ij), the reference's
 * cross_entropy_prob_kernel (CrossEntropyLossKernel.cu:532-576: row max, the
 * sum of exp, log_denom = log(sum) + max, then sum_j t_j (log_denom - x_j))
 * and upstream's cross_entropy_loss_prob_target -(log_softmax(x) * t);
 * mean divides the row sum by n (NaN for n = 0).  lse_i and
 * tsum_i = sum_j t_ij are returned for the gradient. */
void or_ce_prob_fwd(const double* x, const double* t, int64_t n, int64_t c, int reduction, double* loss,
                    double* lse, double* tsum) {
  double sum = 0.0;
  for (int64_t i = 0; i < n; ++i) {
    const double* r = x + i * c;
    const double* tr = t + i * c;
    double m = -INFINITY;
    for (int64_t j = 0; j < c; ++j) m = r[j] > m ? r[j] : m;
    double s = 0.0, T = 0.0, l = 0.0;
    for (int64_t j = 0; j < c; ++j) s += exp(r[j] - m);
    const double ld = m + log(s);
    for (int64_t j = 0; j < c; ++j) {
      l += tr[j] * (ld - r[j]);
      T += tr[j];
    }
    lse[i] = ld;
    tsum[i] = T;
    if (reduction == 0) loss[i] = l;
    sum += l;
  }
  if (reduction == 1) loss[0] = sum / (double)n;
  else if (reduction == 2) loss[0] = sum;
}

/* Its gradient w.r.t. x: g_i (exp(x_ij - lse_i) tsum_i - t_ij), g_i = g[i]
 * (none), g / n (mean), g (sum): the reference's prob_target backward
 * (CrossEntropyLoss.cpp:94-131), grad_lp = -t g_i through
 * _log_softmax_backward_data (grad_lp - softmax * sum_j grad_lp). */
void or_ce_prob_bwd(const double* g, const double* x, const double* t, const double* lse, const double* tsum,
                    int64_t n, int64_t c, int reduction, double* gx) {
  for (int64_t i = 0; i < n; ++i) {
    const double gi = reduction == 0 ? g[i] : (reduction == 1 ? g[0] / (double)n : g[0]);
    const double* r = x + i * c;
    const double* tr = t + i * c;
    double* o = gx + i * c;
    for (int64_t j = 0; j < c; ++j) o[j] = (exp(r[j] - lse[i]) * tsum[i] - tr[j]) * gi;
  }
}

/* ------------------------------------------------------------- losses -- */

enum { OR_MSE = 0, OR_SMOOTH_L1 = 1, OR_BCE_LOGITS = 2 };

/* Pointwise loss terms (float32 opmath):
 *  mse:        d = x - t; d*d                                   (NF:11832)
 *  smooth_l1:  z = |x - t|; z < beta ? 0.5*z*z/beta : z - 0.5*beta   (NF:11988)
 *  bce_logits: (1-t)*x + lw*(m + log(exp(-m) + exp(-x-m))),
 *              m = max(-x, 0), lw = (pw-1)*t + 1
 *              (BinaryCrossEntropyWithLogitsKernel.cu:17-35).  exp(-m) and
 *              exp(-x-m) are 1 and exp(-|x|) in some order, so the sum is
 *              1 + exp(-|x|) exactly as the reference forms it.  Without
 *              pos_weight the reference's other variant applies:
 *              (1-t)*x + m + log(...) (same file :17-23). */
static inline float loss_term(int op, float x, float t, int has_pw, float pw, float beta) {
  switch (op) {
    case OR_MSE: { const float d = x - t; return d * d; }
    case OR_SMOOTH_L1: {
      const float z = fabsf(x - t);
      return z < beta ? ((0.5f * z) * z) / beta : z - 0.5f * beta;
    }
    default: {
      const float m = x < 0.0f ? -x : 0.0f;
      const float lse = or_logf(1.0f + or_expf(-fabsf(x)));
      if (!has_pw) return fmaf(1.0f - t, x, m) + lse;
      const float lw = fmaf(pw - 1.0f, t, 1.0f);
      return fmaf(1.0f - t, x, lw * (m + lse));
    }
  }
}

/* Loss forward.  pw (pos_weight, already broadcast to n elements) and w
 * (weight) may be NULL.  reduction 0 none -> out[n]; 1 mean / 2 sum -> out[0],
 * summed in double (the reference materialises the loss then calls
 * loss.mean()/loss.sum(): BinaryCrossEntropyWithLogits.cpp:63-72). */
void or_loss_fwd(int op, const float* x, const float* t, const float* pw, const float* w,
                 int64_t n, int reduction, float beta, float* out) {
  double acc = 0.0;
  for (int64_t i = 0; i < n; ++i) {
    float v = loss_term(op, x[i], t[i], pw != NULL, pw ? pw[i] : 1.0f, beta);
    if (w) v = v * w[i];
    if (reduction == 0) out[i] = v; else acc += (double)v;
  }
  if (reduction == 1) out[0] = (float)(acc / (double)n);
  else if (reduction == 2) out[0] = (float)acc;
}

/* Loss backward (g is grad_output: n elements for 'none', 1 otherwise):
 *  mse:        ((x - t) * norm) * g, norm = float(2/n) for mean else 2   (NF:11846)
 *  smooth_l1:  d = x - t; d < -beta ? -norm*g : d > beta ? norm*g : norm*d*g/beta,
 *              norm = float(1/n) for mean else 1                         (NF:12002)
 *  bce_logits: the autograd formula's op sequence
 *              (torchgen/packaged/autograd/derivatives.yaml:2017-2019):
 *              u = pw*t; ((u + 1 - t) * sigmoid(x) - u) * g [* w] [/ n]. */
void or_loss_bwd(int op, const float* g, const float* x, const float* t, const float* pw,
                 const float* w, int64_t n, int reduction, float beta, float* gin) {
  const float norm_mse = reduction == 1 ? (float)(2.0 / (double)n) : 2.0f;
  const float norm_l1 = reduction == 1 ? (float)(1.0 / (double)n) : 1.0f;
  for (int64_t i = 0; i < n; ++i) {
    const float gi = reduction == 0 ? g[i] : g[0];
    float r;
    switch (op) {
      case OR_MSE: r = ((x[i] - t[i]) * norm_mse) * gi; break;
      case OR_SMOOTH_L1: {
        const float d = x[i] - t[i];
        r = d < -beta ? (-norm_l1) * gi : (d > beta ? norm_l1 * gi : ((norm_l1 * d) * gi) / beta);
        break;
      }
      default: {
        const float s = act_fwd(OR_SIGMOID, x[i]);
        if (pw) {
          const float u = pw[i] * t[i];
          r = ((u + 1.0f) - t[i]) * s - u;
        } else {
          r = s - t[i];
        }
        r = r * gi;
        if (w) r = r * w[i];
        if (reduction == 1) r = r / (float)n;
        break;
      }
    }
    gin[i] = r;
  }
}

/* --------------------------------------------------------------- AMP -- */

/* _amp_foreach_non_finite_check_and_unscale_ (AmpKernels.cu): x *= inv_scale
 * in place unless inv_scale is exactly 1; returns 1 if any element was inf or
 * NaN before the multiply. */
int or_amp_unscale_f32(float* x, int64_t n, float inv_scale) {
  int bad = 0;
  for (int64_t i = 0; i < n; ++i) {
    if (!isfinite(x[i])) bad = 1;
    x[i] = inv_scale == 1.0f ? x[i] : x[i] * inv_scale;
  }
  return bad;
}

/* _amp_update_scale_ (AmpKernels.cu): backoff on overflow, growth after
 * growth_interval successful steps; products in double rounded to float. */
void or_amp_update_scale(float* scale, int32_t* tracker, float found_inf, double growth, double backoff,
                         int64_t interval) {
  if (found_inf != 0.0f) {
    *scale = (float)((double)*scale * backoff);
    *tracker = 0;
  } else {
    const int64_t successful = (int64_t)*tracker + 1;
    if (successful == interval) {
      const float grown = (float)((double)*scale * growth);
      if (isfinite(grown)) *scale = grown;
      *tracker = 0;
    } else {
      *tracker = (int32_t)successful;
    }
  }
}

/* ----------------------------------------------------------- reductions -- */

/* sum / mean over all elements (ReduceSumKernel.cu:102-113,
 * ReduceMomentKernel.cu:37-55): accumulate in double here. */
double or_sum_f32(const float* x, int64_t n) {
  double s = 0.0;
  for (int64_t i = 0; i < n; ++i) s += (double)x[i];
  return s;
}

/* ------------------------------------------------------------ optimizer -- */

/* beta^step for the integral step counts the optimizer keeps (state_steps
 * holds 1, 2, 3, ... as float): square-and-multiply in double; the device
 * evaluates the same sequence. */
static double pow_int_steps(double beta, float step) {
  double r = 1.0, b = beta;
  uint64_t k = (uint64_t)step;
  if ((float)k != step) return pow(beta, (double)step);
  while (k) { if (k & 1u) r *= b; b *= b; k >>= 1; }
  return r;
}

/* One _fused_adamw_ step over one tensor (NF:16041), the order of operations
 * of upstream adam_math in ADAMW mode
 * (torch/include/ATen/native/cuda/fused_adam_utils.cuh:27-93, step and bias
 * correction :130-137): hyper-parameters are double, state is float, and each
 * mixed expression is evaluated in double and rounded once to float.  The
 * double expressions are written with the fused multiply-adds the device
 * compiler forms for them, so the float results match bit for bit.  l2 = 1:
 * _fused_adam_ (NF:16021), ADAM_MODE::ORIGINAL, the weight decay added to
 * the gradient (fused_adam_utils.cuh:49-51). */
void or_adamw_step(float* p, float* g, float* m, float* v, int64_t n, float step,
                   double lr, double beta1, double beta2, double weight_decay, double eps,
                   int maximize, const float* grad_scale, int amsgrad, float* vmax, int l2) {
  const float bc1 = (float)(1.0 - pow_int_steps(beta1, step));
  const float bc2_sqrt = (float)sqrt(1.0 - pow_int_steps(beta2, step));
  const float step_size = (float)(lr / (double)bc1);
  const double lr_wd = lr * weight_decay;
  for (int64_t i = 0; i < n; ++i) {
    float param = p[i];
    float grad = g[i];
    if (grad_scale) grad = (float)((double)grad / (double)(*grad_scale));
    const float grad_to_store = grad;
    if (maximize) grad = -grad;
    float ea = m[i], eas = v[i];
    if (weight_decay != 0.0) {
      if (l2) grad = (float)((double)grad + (double)param * weight_decay); /* ADAM_MODE::ORIGINAL */
      else param = (float)fma(-lr_wd, (double)param, (double)param);
    }
    ea = (float)fma(beta1, (double)ea, (1.0 - beta1) * (double)grad);
    eas = (float)fma(beta2, (double)eas, ((1.0 - beta2) * (double)grad) * (double)grad);
    float denom;
    if (amsgrad) {
      const float mx = vmax[i] > eas ? vmax[i] : eas;
      vmax[i] = mx;
      denom = (float)((double)(sqrtf(mx) / bc2_sqrt) + eps);
    } else {
      denom = (float)((double)(sqrtf(eas) / bc2_sqrt) + eps);
    }
    param = param - (step_size * ea) / denom;
    p[i] = param;
    if (grad_scale) g[i] = grad_to_store;
    m[i] = ea;
    v[i] = eas;
  }
}

/* _fused_sgd_ step (upstream sgd_math, FusedSgdKernel.cu; the reference
 * registers upstream's kernel): float32 state, double hyper-parameters, each
 * mixed expression in double with a + b c as one fma, rounded once.  buf is
 * NULL without momentum; `first` writes it with the gradient.  The double
 * buffer value feeds the nesterov step before its rounding for storage. */
void or_sgd_step(float* p, float* g, float* buf, int64_t n, double weight_decay, double momentum, double lr,
                 double dampening, int nesterov, int maximize, int first, const float* grad_scale) {
  for (int64_t i = 0; i < n; ++i) {
    float param = p[i];
    float grad = g[i];
    if (grad_scale) {
      grad = (float)((double)grad / (double)(*grad_scale));
      g[i] = grad;
    }
    if (maximize) grad = -grad;
    if (weight_decay != 0.0) grad = (float)fma(weight_decay, (double)param, (double)grad);
    if (buf) {
      const double b = first ? (double)grad : fma(momentum, (double)buf[i], (1.0 - dampening) * (double)grad);
      buf[i] = (float)b;
      grad = nesterov ? (float)fma(momentum, b, (double)grad) : (float)b;
    }
    p[i] = (float)fma(-lr, (double)grad, (double)param);
  }
}

/* ------------------------------------------------------ random numbers -- */

/* Philox4x32-10 (Salmon, Moraes, Dror, Shaw, "Parallel random numbers: as
 * easy as 1, 2, 3", SC 2011): ten rounds of the two 32x32->64 multiplies
 * (0xD2511F53, 0xCD9E8D57), the key bumped by the Weyl constants
 * (0x9E3779B9, 0xBB67AE85) between rounds.  Pinned by the Random123
 * known-answer vectors in tests/test_oracle_rng.py. */
void or_philox4x32_10(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4]) {
  uint32_t c0 = ctr[0], c1 = ctr[1], c2 = ctr[2], c3 = ctr[3], k0 = key[0], k1 = key[1];
  for (int r = 0; r < 10; ++r) {
    if (r) { k0 += 0x9E3779B9u; k1 += 0xBB67AE85u; }
    const uint64_t p0 = (uint64_t)0xD2511F53u * c0, p1 = (uint64_t)0xCD9E8D57u * c2;
    const uint32_t n0 = (uint32_t)(p1 >> 32) ^ c1 ^ k0, n2 = (uint32_t)(p0 >> 32) ^ c3 ^ k1;
    c1 = (uint32_t)p1;
    c3 = (uint32_t)p0;
    c0 = n0;
    c2 = n2;
  }
  out[0] = c0; out[1] = c1; out[2] = c2; out[3] = c3;
}

/* The device's element stream: element i is word i % 4 of
 * philox(counter = (i / 4 as 64 bits, offset as 64 bits), key = seed). */
void or_rng_u32(uint64_t seed, uint64_t offset, int64_t n, uint32_t* out) {
  const uint32_t key[2] = {(uint32_t)seed, (uint32_t)(seed >> 32)};
  for (int64_t q = 0; q * 4 < n; ++q) {
    const uint32_t ctr[4] = {(uint32_t)q, (uint32_t)((uint64_t)q >> 32), (uint32_t)offset, (uint32_t)(offset >> 32)};
    uint32_t r[4];
    or_philox4x32_10(ctr, key, r);
    for (int j = 0; j < 4 && q * 4 + j < n; ++j) out[q * 4 + j] = r[j];
  }
}

/* u in [0, 1) from the top 24 bits of a word. */
static inline float or_u01(uint32_t r) { return (float)(r >> 8) * 5.9604644775390625e-08f; }

/* uniform_(from, to): fma(u, to - from, from) in float, with `to - from`
 * rounded to float first (float32 storage; the front end rounds to a 16-bit
 * storage type and maps a value equal to `to` back to `from`, as upstream's
 * uniform_kernel does). */
void or_uniform_f32(uint64_t seed, uint64_t offset, int64_t n, float lo, float hi, uint32_t* scratch, float* out) {
  or_rng_u32(seed, offset, n, scratch);
  const float range = hi - lo;
  for (int64_t i = 0; i < n; ++i) out[i] = fmaf(or_u01(scratch[i]), range, lo);
}

/* normal_(mean, std): Box-Muller in double on the word pairs (0, 1) and
 * (2, 3) of each Philox call; u1 = (hi24 + 1) 2^-24 in (0, 1], u2 = hi24
 * 2^-24; r = sqrt(-2 log u1), t = 2 pi u2; z = r cos t, r sin t;
 * out = (float)(mean + std z); a 16-bit storage type rounds that float
 * once more.  (The device evaluates sin / cos as
 * sincospi(2 u2); the two differ by rounding far below float precision.) */
void or_normal_f32(uint64_t seed, uint64_t offset, int64_t n, double mean, double stdv, float* out) {
  const double pi = 3.14159265358979323846;
  const uint32_t key[2] = {(uint32_t)seed, (uint32_t)(seed >> 32)};
  for (int64_t q = 0; q * 4 < n; ++q) {
    const uint32_t ctr[4] = {(uint32_t)q, (uint32_t)((uint64_t)q >> 32), (uint32_t)offset, (uint32_t)(offset >> 32)};
    uint32_t r[4];
    or_philox4x32_10(ctr, key, r);
    double z[4];
    for (int h = 0; h < 2; ++h) {
      const double u1 = ((double)(r[2 * h] >> 8) + 1.0) * 5.9604644775390625e-08;
      const double u2 = (double)(r[2 * h + 1] >> 8) * 5.9604644775390625e-08;
      const double rr = sqrt(-2.0 * log(u1));
      z[2 * h] = rr * cos(2.0 * pi * u2);
      z[2 * h + 1] = rr * sin(2.0 * pi * u2);
    }
    for (int j = 0; j < 4 && q * 4 + j < n; ++j) out[q * 4 + j] = (float)(mean + stdv * z[j]);
  }
}

/* dropout with keep probability q: mask = u < q; out = (x * mask) * scale,
 * scale = 1.0 / q divided in double and rounded to float (upstream
 * Dropout.cu fused_dropout_kernel: accscalar_t scale = 1.0 / p). */
void or_dropout_f32(uint64_t seed, uint64_t offset, int64_t n, const float* x, float q, uint32_t* scratch,
                    float* out, uint8_t* mask) {
  or_rng_u32(seed, offset, n, scratch);
  const float scale = (float)(1.0 / (double)q);
  for (int64_t i = 0; i < n; ++i) {
    const int keep = or_u01(scratch[i]) < q;
    mask[i] = (uint8_t)keep;
    out[i] = (x[i] * (keep ? 1.0f : 0.0f)) * scale;
  }
}
