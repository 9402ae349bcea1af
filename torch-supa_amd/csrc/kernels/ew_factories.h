// Op factories shared by the elementwise translation units.
#pragma once

#include <cmath>

#include "ew_launch.h"
#include "ops.h"

namespace sa {

template <template <typename> class Op, bool FloatOnly = false>
struct SimpleFactory {
  template <typename C> static constexpr bool ok() { return !FloatOnly || std::is_floating_point<C>::value; }
  template <typename C> Op<C> make() const { return Op<C>{}; }
};

// trunc division with the 16-bit storage type it rounds its quotient to
struct DivTruncFactory {
  int rt;
  template <typename C> static constexpr bool ok() { return true; }
  template <typename C> DivTruncOp<C> make() const {
    DivTruncOp<C> o{};
    o.rt = rt;
    return o;
  }
};

struct AddFactory {
  double alpha;
  int64_t ialpha;
  template <typename C> static constexpr bool ok() { return true; }
  template <typename C> AddOp<C> make() const {
    if constexpr (std::is_floating_point<C>::value) return AddOp<C>{static_cast<C>(alpha)};
    else if constexpr (std::is_same<C, bool>::value) return AddOp<C>{ialpha != 0 || alpha != 0.0};
    else return AddOp<C>{static_cast<C>(ialpha)};
  }
};

template <int K, bool Bwd>
struct UnaryFactory {
  template <typename C> static constexpr bool ok() {
    if constexpr (Bwd) return std::is_floating_point<C>::value;
    else if constexpr (K == U_RELU || K == U_NEG || K == U_ABS || K == U_SIGN || K == U_FLOOR || K == U_CEIL ||
                       K == U_ROUND || K == U_TRUNC)
      return true;
    else if constexpr (K == U_BITNOT) return std::is_integral<C>::value;
    else return std::is_floating_point<C>::value;
  }
  template <typename C> auto make() const {
    if constexpr (Bwd) return UnaryBwdOp<K, C>{};
    else return UnaryOp<K, C>{};
  }
};

template <int K>
struct BitFactory {
  template <typename C> static constexpr bool ok() { return std::is_integral<C>::value; }
  template <typename C> BitOp<K, C> make() const { return BitOp<K, C>{}; }
};
template <int K>
struct LogicalFactory {
  template <typename C> static constexpr bool ok() { return true; }
  template <typename C> LogicalOp<K, C> make() const { return LogicalOp<K, C>{}; }
};
struct PowScalarFactory {
  int mode, half;
  double e;
  template <typename C> static constexpr bool ok() { return std::is_floating_point<C>::value; }
  template <typename C> PowScalarOp<C> make() const { return PowScalarOp<C>{mode, half, e}; }
};

template <int K, bool Bwd>
int run_unary(const supa_amd_ew_desc* d, void* stream) {
  return run_ew(UnaryFactory<K, Bwd>{}, d, stream, Bwd ? 3 : 2);
}

struct MseBwdFactory {
  double norm;
  int half;
  template <typename C> static constexpr bool ok() { return std::is_floating_point<C>::value; }
  template <typename C> MseBwdOp<C> make() const { return MseBwdOp<C>{storage_param<C>(norm, half), half}; }
};
struct SmoothL1BwdFactory {
  double norm, beta;
  int half;
  template <typename C> static constexpr bool ok() { return std::is_floating_point<C>::value; }
  template <typename C> SmoothL1BwdOp<C> make() const {
    return SmoothL1BwdOp<C>{storage_param<C>(norm, half), storage_param<C>(beta, half), half};
  }
};

struct HuberBwdFactory {
  double norm, delta;
  int half;
  template <typename C> static constexpr bool ok() { return std::is_floating_point<C>::value; }
  template <typename C> HuberBwdOp<C> make() const {
    return HuberBwdOp<C>{storage_param<C>(norm, half), storage_param<C>(delta, half), half};
  }
};
template <bool W>
struct BceProbBwdFactory {
  double div;
  int half;
  template <typename C> static constexpr bool ok() { return std::is_floating_point<C>::value; }
  template <typename C> BceProbBwdOp<W, C> make() const { return BceProbBwdOp<W, C>{static_cast<C>(div), half}; }
};

template <template <typename> class Op, bool FloatOnly = false>
struct ValueFactory {  // ternary ops with one bound value (addcmul, addcdiv)
  double value;
  int64_t ivalue;
  template <typename C> static constexpr bool ok() { return !FloatOnly || std::is_floating_point<C>::value; }
  template <typename C> Op<C> make() const {
    if constexpr (std::is_floating_point<C>::value) return Op<C>{static_cast<C>(value)};
    else if constexpr (std::is_same<C, bool>::value) return Op<C>{ivalue != 0 || value != 0.0};
    else return Op<C>{static_cast<C>(ivalue)};
  }
};

template <int K, bool Bwd>
struct ActFactory {
  double p0, p1, p2;
  int flag;
  template <typename C> static constexpr bool ok() {
    if constexpr (K == A_THRESHOLD && !Bwd) return !std::is_same<C, bool>::value;
    else return std::is_floating_point<C>::value;
  }
  template <typename C> auto make() const {
    if constexpr (Bwd) return ActBwdOp<K, C>{static_cast<C>(p0), static_cast<C>(p1), static_cast<C>(p2), flag};
    else return ActOp<K, C>{static_cast<C>(p0), static_cast<C>(p1), static_cast<C>(p2)};
  }
};

template <bool PW, bool W>
struct BceBwdFactory {
  double n;
  int mean, rt;
  template <typename C> static constexpr bool ok() { return std::is_floating_point<C>::value; }
  template <typename C> BceBwdOp<PW, W, C> make() const {
    const bool pow2 = n >= 1.0 && std::ldexp(1.0, std::ilogb(n)) == n;
    return BceBwdOp<PW, W, C>{static_cast<C>(n), mean, rt, pow2 ? static_cast<C>(1.0 / n) : C(0)};
  }
};

}  // namespace sa
