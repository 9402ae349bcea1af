// Op functors of the elementwise path.  Each functor computes one element in
// the compute type C (float for float32/bfloat16/float16, double, int64 for
// integers, bool) and keeps the operation order of the reference functor it
// replaces, so a float32 result is reproducible bit for bit.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "devmath.h"

namespace sa {

template <typename C> constexpr bool is_fp() { return std::is_floating_point<C>::value; }

// a * b + c with one rounding for floating types (the contraction the
// reference's compiler applies to `self + alpha * other`).
template <typename C> __device__ __forceinline__ C muladd(C a, C b, C c) {
  if constexpr (std::is_same<C, float>::value) return fmaf(a, b, c);
  else if constexpr (std::is_same<C, double>::value) return fma(a, b, c);
  else if constexpr (std::is_same<C, bool>::value) return c || (a && b);
  else return (C)((uint64_t)c + (uint64_t)a * (uint64_t)b);  // wrapping
}

// ------------------------------------------------------------- binary
// add: ufunc::add `self + alpha * other` (UfuncCUDA_add.cu:13-16).
template <typename C> struct AddOp {
  static constexpr bool kLowpMix = true;
  static constexpr int arity = 2;
  C alpha;
  __device__ __forceinline__ C operator()(const C* x) const { return muladd<C>(alpha, x[1], x[0]); }
};
// mul: MulFunctor (BinaryInternal.h:17-30; bool is &&).
template <typename C> struct MulOp {
  static constexpr bool kLowpMix = true;
  static constexpr int arity = 2;
  __device__ __forceinline__ C operator()(const C* x) const {
    if constexpr (std::is_same<C, bool>::value) return x[0] && x[1];
    else if constexpr (std::is_integral<C>::value) return (C)((uint64_t)x[0] * (uint64_t)x[1]);
    else return x[0] * x[1];
  }
};
// true division: DivFunctor `a / b` (BinaryInternal.h:10-15), IEEE.
template <typename C> struct DivTrueOp {
  static constexpr bool kLowpMix = true;
  static constexpr int arity = 2;
  __device__ __forceinline__ C operator()(const C* x) const { return x[0] / x[1]; }
};
// trunc division (BinaryDivTruncKernel.cu:22-55): std::trunc(a / b) on the
// storage type, so for bf16 / f16 tensor operands the quotient is rounded to
// that type before it is truncated (rt 1: bf16, 2: f16; c10's 16-bit division
// computes in float and rounds).  An immediate (CPU-scalar) divisor takes
// rt 0: the float quotient is truncated, as the reference's is_cpu_scalar
// branch (:30-41) and upstream CPU do; the quotient is the IEEE a / b, where
// that branch multiplies by a float reciprocal (the same choice as true
// division's, for bit-exact agreement with the CPU).  Integer division by
// zero has no defined value on the device; it yields 0 here.
template <typename C> struct DivTruncOp {
  static constexpr int arity = 2;
  int rt = 0;
  __device__ __forceinline__ C operator()(const C* x) const {
    if constexpr (std::is_floating_point<C>::value) {
      C q = x[0] / x[1];
      if constexpr (std::is_same<C, float>::value) {
        if (rt == 1) q = bf16_to_f32(f32_to_bf16(q));
        if (rt == 2) q = (float)f32_to_f16(q);
      }
      return trunc(q);
    } else if constexpr (std::is_same<C, bool>::value) {
      return x[0];
    } else {
      return x[1] == 0 ? C(0) : x[0] / x[1];
    }
  }
};
// floor division with Python semantics: c10::div_floor_floating /
// c10::div_floor_integer (BinaryDivFloorKernel.cu:22-82).
template <typename C> struct DivFloorOp {
  static constexpr int arity = 2;
  __device__ __forceinline__ C operator()(const C* x) const {
    const C a = x[0], b = x[1];
    if constexpr (std::is_floating_point<C>::value) {
      if (b == C(0)) return a / b;
      const C mod = fmod(a, b);
      C div = (a - mod) / b;
      if (mod != C(0) && ((b < C(0)) != (mod < C(0)))) div -= C(1);
      C fl;
      if (div != C(0)) {
        fl = floor(div);
        if (div - fl > C(0.5)) fl += C(1);
      } else {
        fl = copysign(C(0), a / b);
      }
      return fl;
    } else if constexpr (std::is_same<C, bool>::value) {
      return a;
    } else {
      if (b == 0) return C(0);
      if ((a < 0) != (b < 0)) {
        const C q = a / b;
        const C r = a % b;
        return r ? q - 1 : q;
      }
      return a / b;
    }
  }
};

// -------------------------------------------------------- activations
// Constants in double; the float kernels use their binary32 roundings.
constexpr double kSqrt1_2 = 0.70710678118654752440;
constexpr double kGeluBetaNone = 0.3989422804014327;  // M_2_SQRTPI * M_SQRT1_2 * 0.5
constexpr double kGeluBetaTanh = 0.7978845608028654;  // M_SQRT2 * M_2_SQRTPI * 0.5
constexpr double kGeluKappa = 0.044715;
static_assert((float)kSqrt1_2 == 0.70710678118654752440f, "constant rounding");
static_assert((float)kGeluBetaNone == 0.3989422804014327f, "constant rounding");
static_assert((float)kGeluBetaTanh == 0.7978845608028654f, "constant rounding");
static_assert((float)kGeluKappa == 0.044715f, "constant rounding");

// gelu in the reference's operation order (upstream GeluKernel.cu, CPU
// Gelu.h:34-41 and 61-65): 'none' (x * 0.5) * (1 + erf(x * sqrt(1/2)));
// 'tanh' (0.5 * x) * (1 + tanh(b * (x + k x^3))), x^3 = (x * x) * x and
// x + k x^3 one fused multiply-add, as the reference's compilers contract it.
template <typename C> __device__ __forceinline__ C gelu_none(C x) {
  // a NaN x makes x * 0.5 NaN, so erf needs no NaN select
  if constexpr (std::is_same<C, float>::value) return (x * 0.5f) * (1.0f + sa_erff_nn(x * (float)kSqrt1_2));
  else return (x * C(0.5)) * (C(1) + erf(x * C(kSqrt1_2)));
}
template <typename C> __device__ __forceinline__ C gelu_tanh(C x) {
  const C x3 = (x * x) * x;
  if constexpr (std::is_same<C, float>::value) {
    const float inner = (float)kGeluBetaTanh * fmaf((float)kGeluKappa, x3, x);
    return (0.5f * x) * (1.0f + sa_tanhf_fast_nn(inner));  // a NaN x makes 0.5 x NaN
  } else {
    const C inner = C(kGeluBetaTanh) * fma(C(kGeluKappa), x3, x);
    return (C(0.5) * x) * (C(1) + tanh(inner));
  }
}
// Opt-in cancellation-free forms (not the reference's arithmetic).  'none':
// x - (x/2) erfc(|x|/sqrt2) for x >= 0, (x/2) erfc(|x|/sqrt2) for x < 0, erfc
// through log erfc (sa_gelu_none); 'tanh': x / (1 + exp(-2u)), u = b (x + k
// x^3), from 0.5 (1 + tanh(u)) = 1 / (1 + exp(-2u)).
template <typename C> __device__ __forceinline__ C gelu_logerfc(C x) {
  if constexpr (std::is_same<C, float>::value) return sa_gelu_none(x);
  else return (x * C(0.5)) * erfc(-x * C(kSqrt1_2));
}
template <typename C> __device__ __forceinline__ C gelu_tanh_logistic(C x) {
  const C x3 = (x * x) * x;
  if constexpr (std::is_same<C, float>::value) {
    const float inner = (-2.0f * (float)kGeluBetaTanh) * fmaf((float)kGeluKappa, x3, x);
    return x / (1.0f + sa_expf_nn(inner));  // a NaN x makes the quotient NaN
  } else {
    const C inner = C(-2.0 * kGeluBetaTanh) * fma(C(kGeluKappa), x3, x);
    return x / (C(1) + exp(inner));
  }
}
template <typename C> __device__ __forceinline__ C expx(C x) {
  if constexpr (std::is_same<C, float>::value) return sa_expf(x);
  else return exp(x);
}
template <typename C> __device__ __forceinline__ C logx(C x) {
  if constexpr (std::is_same<C, float>::value) return sa_logf(x);
  else return log(x);
}
template <typename C> __device__ __forceinline__ C tanhx(C x) {
  if constexpr (std::is_same<C, float>::value) return sa_tanhf(x);
  else return tanh(x);
}
template <typename C> __device__ __forceinline__ C erfx(C x) {
  if constexpr (std::is_same<C, float>::value) return sa_erff(x);
  else return erf(x);
}
template <typename C> __device__ __forceinline__ C expm1x(C x) {
  if constexpr (std::is_same<C, float>::value) return sa_expm1f(x);
  else return expm1(x);
}
template <typename C> __device__ __forceinline__ C log1px(C x) {
  if constexpr (std::is_same<C, float>::value) return sa_log1pf(x);
  else return log1p(x);
}
template <typename C> __device__ __forceinline__ C sigmoidx(C x) { return C(1) / (C(1) + expx<C>(-x)); }

enum UnaryKind {
  U_GELU = 0, U_GELU_TANH, U_SILU, U_SIGMOID, U_TANH, U_EXP, U_LOG, U_ERF, U_RELU, U_NEG, U_RECIPROCAL, U_ABS, U_SQRT,
  U_EXPM1, U_LOG1P, U_SIGN, U_FLOOR, U_CEIL, U_ROUND, U_TRUNC, U_RSQRT, U_BITNOT, U_GELU_LOGERFC,
  U_GELU_TANH_LOGISTIC
};

template <int K, typename C> struct UnaryOp {
  static constexpr int arity = 1;
  // binary64 tanh core: arithmetic about as long as the memory time (the erf
  // activations keep one vector per thread: their ranges are branches, and
  // with two vectors live across them c1 gelu measured slower)
  static constexpr bool kHeavy = std::is_same<C, float>::value && (K == U_GELU_TANH || K == U_TANH);
  __device__ __forceinline__ C operator()(const C* v) const {
    const C x = v[0];
    if constexpr (K == U_GELU) return gelu_none<C>(x);
    else if constexpr (K == U_GELU_TANH) return gelu_tanh<C>(x);
    else if constexpr (K == U_GELU_LOGERFC) return gelu_logerfc<C>(x);
    else if constexpr (K == U_GELU_TANH_LOGISTIC) return gelu_tanh_logistic<C>(x);
    else if constexpr (K == U_SILU) {
      if constexpr (std::is_same<C, float>::value) return x / (1.0f + sa_expf_nn(-x));  // NaN x: NaN quotient
      else return x / (C(1) + expx<C>(-x));
    }
    else if constexpr (K == U_SIGMOID) return sigmoidx<C>(x);
    else if constexpr (K == U_TANH) return tanhx<C>(x);
    else if constexpr (K == U_EXP) return expx<C>(x);
    else if constexpr (K == U_LOG) return logx<C>(x);
    else if constexpr (K == U_ERF) return erfx<C>(x);
    else if constexpr (K == U_RELU) {
      if constexpr (std::is_same<C, bool>::value) return x;
      else if constexpr (std::is_floating_point<C>::value) return (x != x) ? x : (x > C(0) ? x : C(0));
      else return x > C(0) ? x : C(0);
    } else if constexpr (K == U_NEG) {
      if constexpr (std::is_same<C, bool>::value) return x;
      else if constexpr (std::is_integral<C>::value) return (C)(0 - (uint64_t)x);
      else return -x;
    } else if constexpr (K == U_RECIPROCAL) {
      return C(1) / x;
    } else if constexpr (K == U_EXPM1) {
      return expm1x<C>(x);
    } else if constexpr (K == U_LOG1P) {
      return log1px<C>(x);
    } else if constexpr (K == U_ABS) {
      if constexpr (std::is_same<C, bool>::value) return x;
      else if constexpr (std::is_integral<C>::value) return x < 0 ? (C)(0 - (uint64_t)x) : x;
      else return fabs(x);
    } else if constexpr (K == U_SIGN) {
      // upstream sign_kernel: (0 < a) - (a < 0); NaN and -0 give +0
      if constexpr (std::is_same<C, bool>::value) return x;
      else return (C)((int)(C(0) < x) - (int)(x < C(0)));
    } else if constexpr (K == U_FLOOR || K == U_CEIL || K == U_ROUND || K == U_TRUNC) {
      if constexpr (!std::is_floating_point<C>::value) return x;  // integers: a copy, as upstream
      else if constexpr (K == U_FLOOR) return floor(x);
      else if constexpr (K == U_CEIL) return ceil(x);
      else if constexpr (K == U_ROUND) return rint(x);  // nearbyint: halves to even
      else return trunc(x);
    } else if constexpr (K == U_RSQRT) {
      return C(1) / sqrt(x);  // IEEE quotient of the correctly rounded root, as upstream CPU
    } else if constexpr (K == U_BITNOT) {
      if constexpr (std::is_same<C, bool>::value) return !x;
      else return ~x;
    } else {
      return sqrt(x);
    }
  }
};

// Backward functors: x[0] = dy, x[1] = forward input (gelu, silu) or forward
// output (sigmoid, tanh); upstream aten activation backward formulas.
template <int K, typename C> struct UnaryBwdOp {
  static constexpr int arity = 2;
  static constexpr bool kHeavy = std::is_same<C, float>::value && K == U_GELU_TANH;
  __device__ __forceinline__ C operator()(const C* v) const {
    const C dy = v[0], x = v[1];
    if constexpr (K == U_GELU || K == U_GELU_LOGERFC) {
      C cdf;
      if constexpr (K == U_GELU_LOGERFC && std::is_same<C, float>::value) cdf = sa_phif(x);
      else if constexpr (std::is_same<C, float>::value) cdf = 0.5f * (1.0f + sa_erff_nn(x * (float)kSqrt1_2));
      else cdf = C(0.5) * (C(1) + erf(x * C(kSqrt1_2)));
      const C pdf = expx<C>((C(-0.5) * x) * x) * C(kGeluBetaNone);
      return dy * muladd<C>(x, pdf, cdf);
    } else if constexpr (K == U_GELU_TANH || K == U_GELU_TANH_LOGISTIC) {
      const C x2 = x * x;
      const C x3 = x2 * x;
      const C inner = C(kGeluBetaTanh) * muladd<C>(C(kGeluKappa), x3, x);
      const C t = tanhx<C>(inner);
      const C left = C(0.5) * x;
      const C right = C(1) + t;
      const C left_d = C(0.5) * right;
      const C right_d = muladd<C>(-t, t, C(1));
      const C three_kappa = std::is_same<C, float>::value ? C(3.0f * (float)kGeluKappa) : C(3.0 * kGeluKappa);
      const C inner_d = C(kGeluBetaTanh) * muladd<C>(three_kappa, x2, C(1));
      return dy * muladd<C>(left * right_d, inner_d, left_d);
    } else if constexpr (K == U_SILU) {
      const C s = C(1) / (C(1) + expx<C>(-x));
      return (dy * s) * muladd<C>(x, C(1) - s, C(1));
    } else if constexpr (K == U_SIGMOID) {
      return (dy * (C(1) - x)) * x;
    } else {
      return dy * muladd<C>(-x, x, C(1));
    }
  }
};

// ------------------------------------------ parameterised activations
// Upstream's CUDA activation functors (ActivationLeakyReluKernel.cu,
// ActivationEluKernel.cu, ActivationSoftplusKernel.cu,
// ActivationHardswishKernel.cu, ActivationHardsigmoidKernel.cu,
// ActivationMishKernel.cu, ActivationLogSigmoidKernel.cu,
// ActivationThresholdKernel.cu) in opmath with the parameters rounded to it;
// `a + b * c` forms are one fma, as that compiler contracts them.  std::max /
// std::min are the device forms (a < b) ? b : a and (b < a) ? b : a.
enum ActKind {
  A_LEAKY_RELU = 0, A_HARDTANH, A_ELU, A_SOFTPLUS, A_HARDSWISH, A_HARDSIGMOID, A_MISH, A_LOG_SIGMOID, A_THRESHOLD,
  A_HARDSHRINK, A_SOFTSHRINK
};
template <typename C> __device__ __forceinline__ C max_lt(C a, C b) { return (a < b) ? b : a; }
template <typename C> __device__ __forceinline__ C min_lt(C a, C b) { return (b < a) ? b : a; }

// p0, p1, p2: leaky_relu (slope); elu (alpha, scale, input_scale); softplus
// (beta, threshold); threshold (threshold, value); hardshrink / softshrink
// (lambda, in scalar_t as upstream's ActivationHardshrinkKernel.cu /
// ActivationSoftshrinkKernel.cu take it: rounded to a 16-bit storage type).
// softshrink keeps a NaN input (its _isnan test); hardshrink's comparisons
// are false for NaN, which passes it through as well.
template <int K, typename C> struct ActOp {
  static constexpr int arity = 1;
  C p0, p1, p2;
  __device__ __forceinline__ C operator()(const C* v) const {
    const C x = v[0];
    if constexpr (K == A_LEAKY_RELU) return x > C(0) ? x : x * p0;
    else if constexpr (K == A_ELU) return x > C(0) ? x * p1 : expm1x<C>(x * p2) * (p0 * p1);
    else if constexpr (K == A_SOFTPLUS) return (x * p0) > p1 ? x : log1px<C>(expx<C>(x * p0)) / p0;
    else if constexpr (K == A_HARDSWISH) return (x * min_lt<C>(max_lt<C>(x + C(3), C(0)), C(6))) * C(1.0f / 6.0f);
    else if constexpr (K == A_HARDSIGMOID) return min_lt<C>(max_lt<C>(x + C(3), C(0)), C(6)) * C(1.0f / 6.0f);
    else if constexpr (K == A_MISH) return x * tanhx<C>(log1px<C>(expx<C>(x)));
    else if constexpr (K == A_LOG_SIGMOID) return min_lt<C>(C(0), x) - log1px<C>(expx<C>(-fabs(x)));
    else if constexpr (K == A_HARDSHRINK) return (x >= -p0 && x <= p0) ? C(0) : x;
    else if constexpr (K == A_SOFTSHRINK) return x != x ? x : (x > p0 ? x - p0 : (x < -p0 ? x + p0 : C(0)));
    else return x <= p0 ? p1 : x;  // threshold
  }
};

// Inputs: the incoming gradient, then the forward input (elu with `flag`: the
// forward output).  hardtanh: p0 = min, p1 = max.
template <int K, typename C> struct ActBwdOp {
  static constexpr int arity = 2;
  C p0, p1, p2;
  int flag;
  __device__ __forceinline__ C operator()(const C* v) const {
    const C g = v[0], x = v[1];
    if constexpr (K == A_LEAKY_RELU) {
      return x > C(0) ? g : g * p0;
    } else if constexpr (K == A_HARDTANH) {
      return (x <= p0 || x >= p1) ? C(0) : g;
    } else if constexpr (K == A_ELU) {
      const C negcoef = p0 * p1;
      if (flag) return x <= C(0) ? (g * p2) * (x + negcoef) : g * p1;
      return x <= C(0) ? ((g * p2) * negcoef) * expx<C>(x * p2) : g * p1;
    } else if constexpr (K == A_SOFTPLUS) {
      const C z = expx<C>(x * p0);
      return (x * p0) > p1 ? g : (g * z) / (z + C(1));
    } else if constexpr (K == A_HARDSWISH) {
      return x < C(-3) ? C(0) : (x <= C(3) ? g * ((x / C(3)) + C(0.5)) : g);
    } else if constexpr (K == A_HARDSIGMOID) {
      return (x > C(-3) && x < C(3)) ? g * C(1.0f / 6.0f) : C(0);
    } else if constexpr (K == A_MISH) {
      const C sg = C(1) / (C(1) + expx<C>(-x));
      const C t = tanhx<C>(log1px<C>(expx<C>(x)));
      return g * muladd<C>(x * sg, muladd<C>(-t, t, C(1)), t);
    } else if constexpr (K == A_LOG_SIGMOID) {
      const bool neg = x < C(0);
      const C z = expx<C>(-fabs(x));
      return g * muladd<C>(neg ? C(-1) : C(1), z / (C(1) + z), neg ? C(1) : C(0));
    } else if constexpr (K == A_HARDSHRINK || K == A_SOFTSHRINK) {
      return (x >= -p0 && x <= p0) ? C(0) : g;  // upstream shrink_backward_kernel
    } else {
      return x <= p0 ? C(0) : g;  // threshold_backward
    }
  }
};

// glu (upstream glu_kernel, ActivationGluKernel.cu): a sigmoid(b) in opmath,
// sigmoid = 1 / (1 + exp(-b)); inputs a, b (the two halves).
template <typename C> struct GluOp {
  static constexpr int arity = 2;
  __device__ __forceinline__ C operator()(const C* v) const {
    const C s = C(1) / (C(1) + expx<C>(-v[1]));
    return v[0] * s;
  }
};
// glu_backward's halves (upstream glu_backward_kernel): the first half's
// gradient sigmoid(b) g (inputs b, g); the second half's ((1 - s) s) g a
// (inputs a, b, g).
template <typename C> struct GluBwdFirstOp {
  static constexpr int arity = 2;
  __device__ __forceinline__ C operator()(const C* v) const {
    const C s = C(1) / (C(1) + expx<C>(-v[0]));
    return s * v[1];
  }
};
template <typename C> struct GluBwdSecondOp {
  static constexpr int arity = 3;
  __device__ __forceinline__ C operator()(const C* v) const {
    const C s = C(1) / (C(1) + expx<C>(-v[1]));
    return (((C(1) - s) * s) * v[2]) * v[0];
  }
};
// prelu (upstream prelu_kernel / prelu_backward_kernel, in scalar_t: one
// operation each, rounded once at the store): x > 0 ? x : w x (inputs x, w);
// the input gradient x > 0 ? g : w g (inputs x, w, g); the elementwise weight
// gradient x > 0 ? 0 : x g (inputs x, g).
template <typename C> struct PreluOp {
  static constexpr int arity = 2;
  __device__ __forceinline__ C operator()(const C* v) const { return v[0] > C(0) ? v[0] : v[1] * v[0]; }
};
template <typename C> struct PreluBwdInputOp {
  static constexpr int arity = 3;
  __device__ __forceinline__ C operator()(const C* v) const { return v[0] > C(0) ? v[2] : v[1] * v[2]; }
};
template <typename C> struct PreluBwdWeightOp {
  static constexpr int arity = 2;
  __device__ __forceinline__ C operator()(const C* v) const { return v[0] > C(0) ? C(0) : v[0] * v[1]; }
};

// ------------------------------------------------------------ ternary
// addcmul / addcdiv: self + value * (t1 op t2), the reference's CUDA
// functors (PointwiseOpsKernel.cu; ForeachPointwiseOp.cu) with `a + v * x`
// contracted into one fma as its compiler does.  inputs: self, t1, t2.
template <typename C> struct AddcmulOp {
  static constexpr int arity = 3;
  C value;
  __device__ __forceinline__ C operator()(const C* x) const {
    if constexpr (std::is_same<C, bool>::value) return x[0] || (value && x[1] && x[2]);
    else return muladd<C>(value, (C)(x[1] * x[2]), x[0]);
  }
};
template <typename C> struct AddcdivOp {
  static constexpr int arity = 3;
  C value;
  __device__ __forceinline__ C operator()(const C* x) const { return muladd<C>(value, x[1] / x[2], x[0]); }
};
// lerp (upstream Lerp.h): |w| < 0.5 ? self + w (end - self)
// : end - (end - self)(1 - w), each product-sum one fma.  inputs: self, end, w.
template <typename C> struct LerpOp {
  static constexpr int arity = 3;
  __device__ __forceinline__ C operator()(const C* x) const {
    const C a = x[0], e = x[1], w = x[2];
    const C d = e - a;
    return fabs(w) < C(0.5) ? muladd<C>(w, d, a) : muladd<C>(-d, C(1) - w, e);
  }
};

// maximum / minimum: a NaN in either operand is the result (upstream
// maximum / minimum kernels); also clamp_min / clamp_max with a bound.
template <typename C> struct MaxOp {
  static constexpr int arity = 2;
  __device__ __forceinline__ C operator()(const C* x) const {
    const C a = x[0], b = x[1];
    if constexpr (std::is_floating_point<C>::value) {
      if (a != a) return a;
      if (b != b) return b;
    }
    return a > b ? a : b;
  }
};
template <typename C> struct MinOp {
  static constexpr int arity = 2;
  __device__ __forceinline__ C operator()(const C* x) const {
    const C a = x[0], b = x[1];
    if constexpr (std::is_floating_point<C>::value) {
      if (a != a) return a;
      if (b != b) return b;
    }
    return a < b ? a : b;
  }
};

// ---------------------------------------------- comparisons and selects
// eq/ne/lt/le/gt/ge in the common dtype (NaN compares unequal to
// everything), 1 or 0 in the compute type; the output is usually bool.
enum CmpKind { CMP_EQ = 0, CMP_NE, CMP_LT, CMP_LE, CMP_GT, CMP_GE };
template <int K, typename C> struct CmpOp {
  static constexpr int arity = 2;
  static constexpr int kDtypeMode = 1;
  __device__ __forceinline__ C operator()(const C* x) const {
    bool r;
    if constexpr (K == CMP_EQ) r = x[0] == x[1];
    else if constexpr (K == CMP_NE) r = x[0] != x[1];
    else if constexpr (K == CMP_LT) r = x[0] < x[1];
    else if constexpr (K == CMP_LE) r = x[0] <= x[1];
    else if constexpr (K == CMP_GT) r = x[0] > x[1];
    else r = x[0] >= x[1];
    return r ? C(1) : C(0);
  }
};
// bitwise and / or / xor on bool and integer storage (computed in bool or
// int64; truncation to the storage width commutes with these ops).
enum BitKind { BIT_AND = 0, BIT_OR, BIT_XOR };
template <int K, typename C> struct BitOp {
  static constexpr int arity = 2;
  __device__ __forceinline__ C operator()(const C* x) const {
    if constexpr (K == BIT_AND) return x[0] & x[1];
    else if constexpr (K == BIT_OR) return x[0] | x[1];
    else return x[0] ^ x[1];
  }
};
// logical and / or / xor / not: operands tested against zero (NaN is
// nonzero), the result 1 or 0 -- a bool output.
enum LogicalKind { LOG_AND = 0, LOG_OR, LOG_XOR, LOG_NOT };
template <int K, typename C> struct LogicalOp {
  static constexpr int arity = K == LOG_NOT ? 1 : 2;
  static constexpr int kDtypeMode = 1;
  __device__ __forceinline__ C operator()(const C* x) const {
    const bool a = x[0] != C(0);
    bool r;
    if constexpr (K == LOG_NOT) {
      r = !a;
    } else {
      const bool b = x[1] != C(0);
      if constexpr (K == LOG_AND) r = a && b;
      else if constexpr (K == LOG_OR) r = a || b;
      else r = a != b;
    }
    return r ? C(1) : C(0);
  }
};
// pow(x, e) for a scalar exponent, floating types, upstream
// pow_tensor_scalar_kernel_impl's cases: e = 2 -> x*x, 3 -> x*x*x, -2 ->
// 1/(x*x) (the quotient in double), otherwise pow in double rounded once.
// `half` = 1 (bf16) / 2 (f16): products are rounded to the storage type
// between factors, as the upstream kernel multiplies in that type.
enum PowMode { POW_GENERAL = 0, POW_SQUARE, POW_CUBE, POW_INV_SQUARE };
template <typename C> struct PowScalarOp {
  static constexpr int arity = 1;
  int mode;
  int half;
  double e;
  __device__ __forceinline__ C rnd(C v) const {
    if constexpr (std::is_same<C, float>::value) {
      if (half == 1) return to_arith(from_arith<bf16>(v));
      if (half == 2) return to_arith(from_arith<f16>(v));
    }
    return v;
  }
  __device__ __forceinline__ C operator()(const C* x) const {
    const C b = x[0];
    if (mode == POW_SQUARE) return b * b;
    if (mode == POW_CUBE) return rnd(b * b) * b;
    if (mode == POW_INV_SQUARE) return (C)(1.0 / (double)rnd(b * b));
    return (C)pow((double)b, e);
  }
};
// pow(base, exponent) elementwise, floating types: pow in double rounded once.
template <typename C> struct PowOp {
  static constexpr int arity = 2;
  __device__ __forceinline__ C operator()(const C* x) const { return (C)pow((double)x[0], (double)x[1]); }
};
template <typename C> struct IsNanOp {
  static constexpr int arity = 1;
  static constexpr int kDtypeMode = 1;
  __device__ __forceinline__ C operator()(const C* x) const { return x[0] != x[0] ? C(1) : C(0); }
};
// native_dropout_backward: (mask * grad) * scale, upstream masked_scale's
// order (a NaN gradient under a zero mask stays NaN there too).
template <typename C> struct MaskScaleOp {
  static constexpr int arity = 2;
  static constexpr int kDtypeMode = 2;
  C scale;
  __device__ __forceinline__ C operator()(const C* x) const { return (x[0] * x[1]) * scale; }
};
// where(cond, a, b) and masked_fill (cond = mask, a = value, b = self).
template <typename C> struct WhereOp {
  static constexpr int arity = 3;
  static constexpr int kDtypeMode = 2;
  __device__ __forceinline__ C operator()(const C* x) const { return x[0] != C(0) ? x[1] : x[2]; }
};

// ------------------------------------------------------------ copy/fill
template <typename C> struct IdentityOp {
  static constexpr int arity = 1;
  static constexpr bool kIdentity = true;  // a same-dtype copy may move the stored bits
  __device__ __forceinline__ C operator()(const C* x) const { return x[0]; }
};

// ------------------------------------------------------ pointwise losses
// round_half(v, half): for a 16-bit storage type (`half` 1 = bf16, 2 = f16)
// v rounded to it; otherwise v.  Upstream's loss kernels compute in
// scalar_t, and an operation between two c10::BFloat16 / c10::Half values
// returns that type (one between such a value and a float returns float), so
// these ops round exactly where that arithmetic does.
template <typename C> __device__ __forceinline__ C round_half(C v, int half) {
  if constexpr (std::is_same<C, float>::value) {
    if (half == 1) return to_arith(from_arith<bf16>(v));
    if (half == 2) return to_arith(from_arith<f16>(v));
  }
  return v;
}
// The 16-bit storage code of storage type T: 1 bf16, 2 f16, 0 otherwise.
template <typename T> constexpr int half_of() {
  return std::is_same<T, bf16>::value ? 1 : (std::is_same<T, f16>::value ? 2 : 0);
}
// round_half with the storage code fixed at compile time (H >= 0: the
// branches fold away) or read from `half` at run time (H < 0).
template <int H, typename C> __device__ __forceinline__ C round_half_t(C v, int half) {
  if constexpr (H < 0) return round_half(v, half);
  else return round_half(v, H);
}
// mse term (upstream mse_kernel_cuda): d = x - t; d * d.  The term itself is
// rounded so that a fused sum adds what the reference's loss tensor holds.
template <typename C, int H = -1> struct MseTermOp {
  static constexpr int arity = 2;
  int half = 0;
  __device__ __forceinline__ C operator()(const C* v) const {
    const C d = round_half_t<H>(v[0] - v[1], half);
    return round_half_t<H>(d * d, half);
  }
};
// smooth_l1 term (upstream smooth_l1_kernel_cuda): z = |x - t| (the
// difference in scalar_t, its magnitude in float); z < beta ? 0.5 z z / beta :
// z - 0.5 beta.  beta and half_beta (0.5 beta) come in scalar_t, i.e. already
// rounded to a 16-bit storage type by the host.
template <typename C, int H = -1> struct SmoothL1TermOp {
  static constexpr int arity = 2;
  C beta, half_beta;
  int half = 0;
  __device__ __forceinline__ C operator()(const C* v) const {
    const C z = fabs(round_half_t<H>(v[0] - v[1], half));
    return round_half_t<H>(z < beta ? ((C(0.5) * z) * z) / beta : z - half_beta, half);
  }
};
// BCE-with-logits term (BinaryCrossEntropyWithLogitsKernel.cu:17-35):
// m = max(-x, 0); exp(-m) + exp(-x-m) is 1 + exp(-|x|) in either order.
// inputs: x, t [, pw] [, w]
// HW: the summed forward (sum / mean) evaluates log(1 + e^-|x|) with the
// hardware base-2 exponential and logarithm (about 1 ulp each); the sum's
// tolerance (rtol 1e-5) covers it, and the per-element (`none`) form keeps
// the exact polynomials the oracle mirrors.
template <bool PW, bool W, typename C, bool HW = false> struct BceTermOp {
  static constexpr int arity = 2 + (PW ? 1 : 0) + (W ? 1 : 0);
  __device__ __forceinline__ C operator()(const C* v) const {
    const C x = v[0], t = v[1];
    const C m = x < C(0) ? -x : C(0);
    C lse;
    if constexpr (std::is_same<C, float>::value && HW)
      lse = 0.693147180559945309f * __builtin_amdgcn_logf(1.0f + __builtin_amdgcn_exp2f(-fabsf(x) * 1.44269504088896341f));
    else if constexpr (std::is_same<C, float>::value)
      lse = sa_logf_normal(1.0f + sa_expf_nn(-fabsf(x)));  // argument in [1, 2]; a NaN x makes r NaN below
    else
      lse = logx<C>(C(1) + expx<C>(-fabs(x)));
    C r;
    if constexpr (PW) {
      const C lw = muladd<C>(v[2] - C(1), t, C(1));
      r = muladd<C>(C(1) - t, x, lw * (m + lse));
    } else {
      r = muladd<C>(C(1) - t, x, m) + lse;
    }
    if constexpr (W) r = r * v[2 + (PW ? 1 : 0)];
    return r;
  }
};
// BCE-with-logits gradient in the autograd formula's op order (inputs g, x,
// t [, pw] [, w]): u = pw * t; ((u + 1) - t) * sigmoid(x) - u, or
// sigmoid(x) - t; * g; * w; / n.  rt: the storage dtype every intermediate is
// rounded to (0 keep C, 1 bf16, 2 f16), as the op-by-op evaluation stores
// each intermediate tensor.  RT / MEAN >= 0 fix rt / mean at compile time
// (the one-vector row-broadcast kernel, k_rowb, launches those forms: with
// the switches read per element the c4 backward ran 3 points slower there).
template <bool PW, bool W, typename C, int RT = -1, int MEAN = -1> struct BceBwdOp {
  static constexpr int arity = 3 + (PW ? 1 : 0) + (W ? 1 : 0);
  static constexpr bool kRowB = true;
  C n;
  int mean;
  int rt;
  // 1 / n when n is a power of two, else 0: r * inv_n and r / n are then the
  // same correctly rounded value (the exact quotient), without the division
  C inv_n;
  template <int R, int M> __device__ __host__ BceBwdOp<PW, W, C, R, M> fixed() const {
    return BceBwdOp<PW, W, C, R, M>{n, mean, rt, inv_n};
  }
  __device__ __forceinline__ C rnd(C v) const {
    if constexpr (std::is_same<C, float>::value) {
      const int r = RT >= 0 ? RT : rt;
      if (r == 1) return bf16_to_f32(f32_to_bf16(v));
      if (r == 2) return (float)f32_to_f16(v);
    }
    return v;
  }
  __device__ __forceinline__ C operator()(const C* v) const {
    const C g = v[0], x = v[1], t = v[2];
    const C s = rnd(sigmoidx<C>(x));
    C r;
    if constexpr (PW) {
      const C u = rnd(v[3] * t);
      r = rnd(rnd(rnd(rnd(u + C(1)) - t) * s) - u);
    } else {
      r = rnd(s - t);
    }
    r = rnd(r * g);
    if constexpr (W) r = rnd(r * v[3 + (PW ? 1 : 0)]);
    if (MEAN >= 0 ? MEAN != 0 : mean != 0) r = inv_n != C(0) ? r * inv_n : r / n;
    return r;
  }
};
// mse backward (upstream mse_backward_cuda_kernel): norm (x - t) g, inputs
// g, x, t; in scalar_t, so every product is rounded for a 16-bit type (norm
// comes rounded to it).
template <typename C> struct MseBwdOp {
  static constexpr int arity = 3;
  // four light streams: k_contig caps residency (the smooth_l1 gradient, with
  // its division, lost 6 points from the same cap)
  static constexpr bool kCapOccupancy = true;
  C norm;
  int half = 0;
  __device__ __forceinline__ C operator()(const C* v) const {
    return round_half(round_half(v[1] - v[2], half) * norm, half) * v[0];
  }
};
// huber (upstream huber_kernel_cuda): z = |a - b|; 0.5 z z below delta,
// delta (z - 0.5 delta) above.
// Rounded for a 16-bit type as the smooth_l1 term (delta and half_delta come
// rounded).
template <typename C, int H = -1> struct HuberTermOp {
  static constexpr int arity = 2;
  C delta, half_delta;
  int half = 0;
  __device__ __forceinline__ C operator()(const C* v) const {
    const C z = fabs(round_half_t<H>(v[0] - v[1], half));
    return round_half_t<H>(z < delta ? (C(0.5) * z) * z : delta * (z - half_delta), half);
  }
};
// huber backward (upstream huber_backward_cuda_kernel), v = {grad, input,
// target}; in scalar_t, every operation rounded for a 16-bit type (norm and
// delta come rounded).
template <typename C> struct HuberBwdOp {
  static constexpr int arity = 3;
  C norm, delta;
  int half = 0;
  __device__ __forceinline__ C operator()(const C* v) const {
    const C g = v[0], x = round_half(v[1] - v[2], half);
    if (x < -delta) return round_half((-norm) * g, half) * delta;
    if (x > delta) return round_half(norm * g, half) * delta;
    return round_half(norm * x, half) * g;
  }
};
// binary_cross_entropy on probabilities (upstream binary_cross_entropy_out
// kernel): (t - 1) max(log1p(-x), -100) - t max(log(x), -100), times the
// weight as a second op; v = {x, t[, w]}.  std::max keeps a NaN log.  For a
// 16-bit storage type every intermediate is rounded to it, as the upstream
// kernel computes in scalar_t.
template <bool W, typename C> struct BceProbTermOp {
  static constexpr int arity = W ? 3 : 2;
  int half;
  __device__ __forceinline__ static C keep_max(C a, C b) { return a < b ? b : a; }
  __device__ __forceinline__ C operator()(const C* v) const {
    const C x = v[0], t = v[1];
    const C lx = keep_max(round_half(logx<C>(x), half), C(-100));
    const C l1mx = keep_max(round_half(log1px<C>(-x), half), C(-100));
    const C a = round_half((round_half(t - C(1), half)) * l1mx, half);
    const C b = round_half(t * lx, half);
    C r = a - b;
    if constexpr (W) r = round_half(r, half) * v[2];
    return r;
  }
};
// its gradient (upstream binary_cross_entropy_backward): g (x - t) /
// max((1 - x) x, 1e-12), then times the weight, then / n for a mean;
// v = {grad, x, t[, w]}, div = n for MEAN else 1; intermediates rounded to a
// 16-bit storage type as in the forward.
template <bool W, typename C> struct BceProbBwdOp {
  static constexpr int arity = W ? 4 : 3;
  C div;
  int half;
  __device__ __forceinline__ C operator()(const C* v) const {
    const C g = v[0], x = v[1], t = v[2];
    const C d0 = round_half(round_half(C(1) - x, half) * x, half);
    const C eps = round_half(C(1e-12), half);
    const C den = d0 < eps ? eps : d0;
    C r = round_half(round_half(g * round_half(x - t, half), half) / den, half);
    if constexpr (W) r = round_half(r * v[3], half);
    return r / div;
  }
};
// xlogy (upstream xlogy_kernel_cuda): NaN for a NaN y, 0 for x == 0, x log y.
template <typename C> struct XlogyOp {
  static constexpr int arity = 2;
  __device__ __forceinline__ C operator()(const C* v) const {
    const C x = v[0], y = v[1];
    if (y != y) return y;
    if (x == C(0)) return C(0);
    return x * logx<C>(y);
  }
};

// smooth_l1 backward (upstream smooth_l1_backward_cuda_kernel), v = {grad,
// input, target}: -norm g below -beta, norm g above beta, norm x g / beta
// between; in scalar_t, every operation rounded for a 16-bit type (norm and
// beta come rounded).
// xlog1py (upstream xlog1py_kernel_cuda): NaN for a NaN y, 0 for x == 0,
// x log1p(y).
template <typename C> struct Xlog1pyOp {
  static constexpr int arity = 2;
  __device__ __forceinline__ C operator()(const C* v) const {
    const C x = v[0], y = v[1];
    if (y != y) return y;
    if (x == C(0)) return C(0);
    return x * log1px<C>(y);
  }
};

template <typename C> struct SmoothL1BwdOp {
  static constexpr int arity = 3;
  C norm, beta;
  int half = 0;
  __device__ __forceinline__ C operator()(const C* v) const {
    const C g = v[0], d = round_half(v[1] - v[2], half);
    return d < -beta ? (-norm) * g
                     : (d > beta ? norm * g : round_half(round_half(norm * d, half) * g, half) / beta);
  }
};

}  // namespace sa
