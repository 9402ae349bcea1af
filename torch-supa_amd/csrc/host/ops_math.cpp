// PrivateUse1 registrations of the pointwise math around the loss path:
// sign / sgn, floor / ceil / round / trunc, rsqrt, the bitwise and logical
// families, xlogy, and pow (tensor ** scalar, tensor ** tensor, scalar **
// tensor)
// -- what losses, normalisations and masks written in plain torch call next
// to the path's ops (label-smoothed cross-entropy builds its kept-row mask
// with bitwise_not, RMS-style norms call pow and rsqrt).  Integer pow takes
// the counted CPU fallback.
#include <ATen/native/CPUFallback.h>
#include <ATen/native/Resize.h>
#include <ATen/ops/pow_ops.h>
#include <torch/library.h>

#include "common.h"
#include "ew_apply.h"

namespace supa {
namespace {

c10::ScalarType default_float_dtype() { return c10::typeMetaToScalarType(c10::get_default_dtype()); }

void check_out_cast(c10::ScalarType common, const at::Tensor& out, const char* name) {
  TORCH_CHECK(c10::canCast(common, out.scalar_type()), name, ": result type ", common,
              " can't be cast to the desired output type ", out.scalar_type());
}

// Runs `fn` with output `out` (in place when `inplace`, a new tensor of
// `result` dtype when `out` is undefined).
at::Tensor apply(const std::vector<EwIn>& ins, c10::ScalarType common, c10::ScalarType result, at::Tensor out,
                 bool inplace, const EwLaunch& fn, const char* name) {
  if (inplace) {
    check_out_cast(result, ins[0].t, name);
    return ew_apply(ins[0].t, ins[0].t.scalar_type(), common, ins, fn, name);
  }
  if (out.defined()) {
    check_out_cast(result, out, name);
    return ew_apply(out, out.scalar_type(), common, ins, fn, name);
  }
  return ew_apply(at::Tensor(), result, common, ins, fn, name);
}

EwLaunch unary_launch(int op) {
  return [op](const supa_amd_ew_desc* d, void* s) { return supa_amd_unary(d, op, s); };
}

// ------------------------------------------------- sign, rounding, rsqrt
at::Tensor unary_any(const at::Tensor& self, at::Tensor out, bool inplace, int op, bool allow_bool, const char* name) {
  TORCH_CHECK(allow_bool || self.scalar_type() != at::kBool, name, ": \"", name, "\" not implemented for 'Bool'");
  TORCH_CHECK(!at::isComplexType(self.scalar_type()), name, ": complex inputs are not supported on supa");
  const c10::ScalarType t = self.scalar_type();
  return apply({EwIn::of(self)}, t, t, out, inplace, unary_launch(op), name);
}

#define SUPA_UNARY_ANY(NAME, OP, ALLOW_BOOL)                                                    \
  at::Tensor pm_##NAME(const at::Tensor& s) { return unary_any(s, {}, false, OP, ALLOW_BOOL, #NAME); } \
  at::Tensor& pm_##NAME##_(at::Tensor& s) {                                                    \
    unary_any(s, {}, true, OP, ALLOW_BOOL, #NAME "_");                                         \
    return s;                                                                                  \
  }                                                                                            \
  at::Tensor& pm_##NAME##_out(const at::Tensor& s, at::Tensor& out) {                          \
    unary_any(s, out, false, OP, ALLOW_BOOL, #NAME ".out");                                 \
    return out;                                                                             \
  }
SUPA_UNARY_ANY(sign, SUPA_AMD_SIGN, true)
SUPA_UNARY_ANY(sgn, SUPA_AMD_SIGN, true)
SUPA_UNARY_ANY(floor, SUPA_AMD_FLOOR, false)
SUPA_UNARY_ANY(ceil, SUPA_AMD_CEIL, false)
SUPA_UNARY_ANY(round, SUPA_AMD_ROUND, false)
SUPA_UNARY_ANY(trunc, SUPA_AMD_TRUNC, false)
#undef SUPA_UNARY_ANY

// rsqrt: integers promote to the default float dtype
at::Tensor rsqrt_into(const at::Tensor& self, at::Tensor out, bool inplace, const char* name) {
  c10::ScalarType common = self.scalar_type();
  if (at::isIntegralType(common, true)) common = default_float_dtype();
  TORCH_CHECK(at::isFloatingType(common), name, ": \"rsqrt\" not implemented for '", common, "'");
  return apply({EwIn::of(self)}, common, common, out, inplace, unary_launch(SUPA_AMD_RSQRT), name);
}
at::Tensor pm_rsqrt(const at::Tensor& s) { return rsqrt_into(s, {}, false, "rsqrt"); }
at::Tensor& pm_rsqrt_(at::Tensor& s) {
  rsqrt_into(s, {}, true, "rsqrt_");
  return s;
}
at::Tensor& pm_rsqrt_out(const at::Tensor& s, at::Tensor& out) {
  rsqrt_into(s, out, false, "rsqrt.out");
  return out;
}

// ----------------------------------------------------------- bitwise
at::Tensor bitwise_not_into(const at::Tensor& self, at::Tensor out, bool inplace, const char* name) {
  const c10::ScalarType t = self.scalar_type();
  TORCH_CHECK(at::isIntegralType(t, true), name, ": \"bitwise_not\" not implemented for '", t, "'");
  return apply({EwIn::of(self)}, t, t, out, inplace, unary_launch(SUPA_AMD_BITWISE_NOT), name);
}
at::Tensor pm_bitwise_not(const at::Tensor& s) { return bitwise_not_into(s, {}, false, "bitwise_not"); }
at::Tensor& pm_bitwise_not_(at::Tensor& s) {
  bitwise_not_into(s, {}, true, "bitwise_not_");
  return s;
}
at::Tensor& pm_bitwise_not_out(const at::Tensor& s, at::Tensor& out) {
  bitwise_not_into(s, out, false, "bitwise_not.out");
  return out;
}

at::Tensor bitwise_into(const at::Tensor& self, const EwIn& other, c10::ScalarType common, at::Tensor out,
                        bool inplace, int op, const char* name) {
  TORCH_CHECK(at::isIntegralType(common, true), name, ": not implemented for '", common, "'");
  const EwLaunch fn = [op](const supa_amd_ew_desc* d, void* s) { return supa_amd_bitwise(d, op, s); };
  return apply({EwIn::of(self), other}, common, common, out, inplace, fn, name);
}
#define SUPA_BITWISE(NAME, OP)                                                                              \
  at::Tensor NAME##_t(const at::Tensor& s, const at::Tensor& o) {                                           \
    return bitwise_into(s, EwIn::of(o), at::result_type(s, o), {}, false, OP, #NAME ".Tensor");             \
  }                                                                                                         \
  at::Tensor& NAME##_t_(at::Tensor& s, const at::Tensor& o) {                                               \
    bitwise_into(s, EwIn::of(o), at::result_type(s, o), {}, true, OP, #NAME "_.Tensor");                    \
    return s;                                                                                               \
  }                                                                                                         \
  at::Tensor& NAME##_t_out(const at::Tensor& s, const at::Tensor& o, at::Tensor& out) {                     \
    bitwise_into(s, EwIn::of(o), at::result_type(s, o), out, false, OP, #NAME ".Tensor_out");               \
    return out;                                                                                             \
  }                                                                                                         \
  at::Tensor NAME##_s(const at::Tensor& s, const c10::Scalar& o) {                                          \
    return bitwise_into(s, EwIn::num(o), at::result_type(s, o), {}, false, OP, #NAME ".Scalar");            \
  }                                                                                                         \
  at::Tensor& NAME##_s_(at::Tensor& s, const c10::Scalar& o) {                                              \
    bitwise_into(s, EwIn::num(o), at::result_type(s, o), {}, true, OP, #NAME "_.Scalar");                   \
    return s;                                                                                               \
  }                                                                                                         \
  at::Tensor& NAME##_s_out(const at::Tensor& s, const c10::Scalar& o, at::Tensor& out) {                    \
    bitwise_into(s, EwIn::num(o), at::result_type(s, o), out, false, OP, #NAME ".Scalar_out");              \
    return out;                                                                                             \
  }
SUPA_BITWISE(bitwise_and, SUPA_AMD_BIT_AND)
SUPA_BITWISE(bitwise_or, SUPA_AMD_BIT_OR)
SUPA_BITWISE(bitwise_xor, SUPA_AMD_BIT_XOR)
#undef SUPA_BITWISE

// ----------------------------------------------------------- logical
// Operands compared against zero in their promoted dtype; the result is bool
// (the out= tensor's dtype for .out, self's for the in-place forms).
at::Tensor logical_into(const std::vector<EwIn>& ins, c10::ScalarType common, at::Tensor out, bool inplace, int op,
                        const char* name) {
  TORCH_CHECK(!at::isComplexType(common), name, ": complex inputs are not supported on supa");
  const EwLaunch fn = [op](const supa_amd_ew_desc* d, void* s) { return supa_amd_logical(d, op, s); };
  return apply(ins, common, at::kBool, out, inplace, fn, name);
}
#define SUPA_LOGICAL(NAME, OP)                                                                            \
  at::Tensor pm_##NAME(const at::Tensor& s, const at::Tensor& o) {                                        \
    return logical_into({EwIn::of(s), EwIn::of(o)}, at::result_type(s, o), {}, false, OP, #NAME);         \
  }                                                                                                       \
  at::Tensor& pm_##NAME##_(at::Tensor& s, const at::Tensor& o) {                                          \
    logical_into({EwIn::of(s), EwIn::of(o)}, at::result_type(s, o), {}, true, OP, #NAME "_");             \
    return s;                                                                                             \
  }                                                                                                       \
  at::Tensor& pm_##NAME##_out(const at::Tensor& s, const at::Tensor& o, at::Tensor& out) {                \
    logical_into({EwIn::of(s), EwIn::of(o)}, at::result_type(s, o), out, false, OP, #NAME ".out");        \
    return out;                                                                                           \
  }
SUPA_LOGICAL(logical_and, SUPA_AMD_LOGICAL_AND)
SUPA_LOGICAL(logical_or, SUPA_AMD_LOGICAL_OR)
SUPA_LOGICAL(logical_xor, SUPA_AMD_LOGICAL_XOR)
#undef SUPA_LOGICAL
at::Tensor pm_logical_not(const at::Tensor& s) {
  return logical_into({EwIn::of(s)}, s.scalar_type(), {}, false, SUPA_AMD_LOGICAL_NOT, "logical_not");
}
at::Tensor& pm_logical_not_(at::Tensor& s) {
  logical_into({EwIn::of(s)}, s.scalar_type(), {}, true, SUPA_AMD_LOGICAL_NOT, "logical_not_");
  return s;
}
at::Tensor& pm_logical_not_out(const at::Tensor& s, at::Tensor& out) {
  logical_into({EwIn::of(s)}, s.scalar_type(), out, false, SUPA_AMD_LOGICAL_NOT, "logical_not.out");
  return out;
}

// --------------------------------------------------------------- pow
// upstream pow_out (Pow.cpp): exponent 0 fills ones, 1 copies; floating
// results route 0.5 / -0.5 / -1 to sqrt / rsqrt / reciprocal
// (pow_tensor_scalar_kernel), the rest to the pow kernel.
at::Tensor& pow_ts_into(const at::Tensor& self, const c10::Scalar& e, at::Tensor& out, const char* name) {
  const c10::ScalarType common = at::result_type(self, e);
  TORCH_CHECK(!at::isComplexType(common), name, ": complex inputs are not supported on supa");
  if (e.equal(0.0)) {
    if (!out.defined()) out = at::empty_like(self, self.options().dtype(common));
    else at::native::resize_output(out, self.sizes());
    out.fill_(1);
    return out;
  }
  if (e.equal(1.0)) {
    if (!out.defined()) out = at::empty_like(self, self.options().dtype(common));
    else at::native::resize_output(out, self.sizes());
    out.copy_(self);
    return out;
  }
  int op = -1;
  if (e.equal(0.5)) op = SUPA_AMD_SQRT;
  else if (e.equal(-0.5)) op = SUPA_AMD_RSQRT;
  else if (e.equal(-1.0)) op = SUPA_AMD_RECIPROCAL;
  EwLaunch fn;
  if (op >= 0) {
    fn = unary_launch(op);
  } else {
    const double ev = e.toDouble();
    fn = [ev](const supa_amd_ew_desc* d, void* s) { return supa_amd_pow_scalar(d, ev, s); };
  }
  out = apply({EwIn::of(self)}, common, common, out, false, fn, name);
  return out;
}

bool pow_native(c10::ScalarType common) { return at::isFloatingType(common); }

at::Tensor pow_ts(const at::Tensor& self, const c10::Scalar& e) {
  if (!pow_native(at::result_type(self, e)))
    return at::native::call_fallback_fn<&supa_cpu_fallback, at::_ops::pow_Tensor_Scalar>::call(self, e);
  at::Tensor out;
  return pow_ts_into(self, e, out, "pow.Tensor_Scalar");
}
at::Tensor& pow_ts_out(const at::Tensor& self, const c10::Scalar& e, at::Tensor& out) {
  if (!pow_native(at::result_type(self, e)))
    return at::native::call_fallback_fn<&supa_cpu_fallback, at::_ops::pow_Tensor_Scalar_out>::call(self, e, out);
  return pow_ts_into(self, e, out, "pow.Tensor_Scalar_out");
}
at::Tensor& pow_ts_(at::Tensor& self, const c10::Scalar& e) {
  if (!pow_native(at::result_type(self, e)))
    return at::native::call_fallback_fn<&supa_cpu_fallback, at::_ops::pow__Scalar>::call(self, e);
  pow_ts_into(self, e, self, "pow_.Scalar");
  return self;
}

EwLaunch pow_launch() {
  return [](const supa_amd_ew_desc* d, void* s) { return supa_amd_pow(d, s); };
}
at::Tensor pow_tt(const at::Tensor& self, const at::Tensor& e) {
  const c10::ScalarType common = at::result_type(self, e);
  if (!pow_native(common))
    return at::native::call_fallback_fn<&supa_cpu_fallback, at::_ops::pow_Tensor_Tensor>::call(self, e);
  return apply({EwIn::of(self), EwIn::of(e)}, common, common, {}, false, pow_launch(), "pow.Tensor_Tensor");
}
at::Tensor& pow_tt_out(const at::Tensor& self, const at::Tensor& e, at::Tensor& out) {
  const c10::ScalarType common = at::result_type(self, e);
  if (!pow_native(common))
    return at::native::call_fallback_fn<&supa_cpu_fallback, at::_ops::pow_Tensor_Tensor_out>::call(self, e, out);
  apply({EwIn::of(self), EwIn::of(e)}, common, common, out, false, pow_launch(), "pow.Tensor_Tensor_out");
  return out;
}
at::Tensor& pow_tt_(at::Tensor& self, const at::Tensor& e) {
  const c10::ScalarType common = at::result_type(self, e);
  if (!pow_native(common))
    return at::native::call_fallback_fn<&supa_cpu_fallback, at::_ops::pow__Tensor>::call(self, e);
  apply({EwIn::of(self), EwIn::of(e)}, common, common, {}, true, pow_launch(), "pow_.Tensor");
  return self;
}
// scalar ** tensor: a base of 1 gives ones (upstream pow(Scalar, Tensor))
at::Tensor& pow_st_into(const c10::Scalar& base, const at::Tensor& e, at::Tensor out, at::Tensor& result,
                        const char* name) {
  const c10::ScalarType common = at::result_type(base, e);
  if (base.equal(1.0)) {
    result = out.defined() ? out : at::empty_like(e, e.options().dtype(common));
    if (out.defined()) at::native::resize_output(result, e.sizes());
    result.fill_(1);
    return result;
  }
  result = apply({EwIn::num(base), EwIn::of(e)}, common, common, out, false, pow_launch(), name);
  return result;
}
at::Tensor pow_st(const c10::Scalar& base, const at::Tensor& e) {
  if (!pow_native(at::result_type(base, e)))
    return at::native::call_fallback_fn<&supa_cpu_fallback, at::_ops::pow_Scalar>::call(base, e);
  at::Tensor r;
  return pow_st_into(base, e, {}, r, "pow.Scalar");
}
at::Tensor& pow_st_out(const c10::Scalar& base, const at::Tensor& e, at::Tensor& out) {
  if (!pow_native(at::result_type(base, e)))
    return at::native::call_fallback_fn<&supa_cpu_fallback, at::_ops::pow_Scalar_out>::call(base, e, out);
  at::Tensor r;
  pow_st_into(base, e, out, r, "pow.Scalar_out");
  return out;
}

// ------------------------------------------------------------- xlogy
// x * log(y) with 0 where x == 0 (kl_div's target log target); integer
// results promote to the default float dtype.
at::Tensor xlogy_into(const EwIn& x, const EwIn& y, c10::ScalarType common, at::Tensor out, bool inplace,
                      const char* name) {
  if (at::isIntegralType(common, true)) common = default_float_dtype();
  TORCH_CHECK(at::isFloatingType(common), name, ": not implemented for '", common, "'");
  const EwLaunch fn = [](const supa_amd_ew_desc* d, void* s) { return supa_amd_xlogy(d, s); };
  return apply({x, y}, common, common, out, inplace, fn, name);
}
// special_xlog1py: x * log1p(y) with the same special cases and promotion
at::Tensor xlog1py_into(const EwIn& x, const EwIn& y, c10::ScalarType common, at::Tensor out, const char* name) {
  if (at::isIntegralType(common, true)) common = default_float_dtype();
  TORCH_CHECK(at::isFloatingType(common), name, ": not implemented for '", common, "'");
  const EwLaunch fn = [](const supa_amd_ew_desc* d, void* s) { return supa_amd_xlog1py(d, s); };
  return apply({x, y}, common, common, out, false, fn, name);
}
at::Tensor xlog1py_t(const at::Tensor& s, const at::Tensor& o) {
  return xlog1py_into(EwIn::of(s), EwIn::of(o), at::result_type(s, o), {}, "special_xlog1py");
}
at::Tensor& xlog1py_t_out(const at::Tensor& s, const at::Tensor& o, at::Tensor& out) {
  xlog1py_into(EwIn::of(s), EwIn::of(o), at::result_type(s, o), out, "special_xlog1py.out");
  return out;
}
at::Tensor xlog1py_so(const at::Tensor& s, const c10::Scalar& o) {
  return xlog1py_into(EwIn::of(s), EwIn::num(o), at::result_type(s, o), {}, "special_xlog1py.other_scalar");
}
at::Tensor& xlog1py_so_out(const at::Tensor& s, const c10::Scalar& o, at::Tensor& out) {
  xlog1py_into(EwIn::of(s), EwIn::num(o), at::result_type(s, o), out, "special_xlog1py.other_scalar_out");
  return out;
}
at::Tensor xlog1py_ss(const c10::Scalar& s, const at::Tensor& o) {
  return xlog1py_into(EwIn::num(s), EwIn::of(o), at::result_type(s, o), {}, "special_xlog1py.self_scalar");
}
at::Tensor& xlog1py_ss_out(const c10::Scalar& s, const at::Tensor& o, at::Tensor& out) {
  xlog1py_into(EwIn::num(s), EwIn::of(o), at::result_type(s, o), out, "special_xlog1py.self_scalar_out");
  return out;
}

at::Tensor xlogy_t(const at::Tensor& s, const at::Tensor& o) {
  return xlogy_into(EwIn::of(s), EwIn::of(o), at::result_type(s, o), {}, false, "xlogy.Tensor");
}
at::Tensor& xlogy_t_out(const at::Tensor& s, const at::Tensor& o, at::Tensor& out) {
  xlogy_into(EwIn::of(s), EwIn::of(o), at::result_type(s, o), out, false, "xlogy.OutTensor");
  return out;
}
at::Tensor& xlogy_t_(at::Tensor& s, const at::Tensor& o) {
  xlogy_into(EwIn::of(s), EwIn::of(o), at::result_type(s, o), {}, true, "xlogy_.Tensor");
  return s;
}
at::Tensor xlogy_so(const at::Tensor& s, const c10::Scalar& o) {
  return xlogy_into(EwIn::of(s), EwIn::num(o), at::result_type(s, o), {}, false, "xlogy.Scalar_Other");
}
at::Tensor& xlogy_so_out(const at::Tensor& s, const c10::Scalar& o, at::Tensor& out) {
  xlogy_into(EwIn::of(s), EwIn::num(o), at::result_type(s, o), out, false, "xlogy.OutScalar_Other");
  return out;
}
at::Tensor& xlogy_so_(at::Tensor& s, const c10::Scalar& o) {
  xlogy_into(EwIn::of(s), EwIn::num(o), at::result_type(s, o), {}, true, "xlogy_.Scalar_Other");
  return s;
}
at::Tensor xlogy_ss(const c10::Scalar& s, const at::Tensor& o) {
  return xlogy_into(EwIn::num(s), EwIn::of(o), at::result_type(s, o), {}, false, "xlogy.Scalar_Self");
}
at::Tensor& xlogy_ss_out(const c10::Scalar& s, const at::Tensor& o, at::Tensor& out) {
  xlogy_into(EwIn::num(s), EwIn::of(o), at::result_type(s, o), out, false, "xlogy.OutScalar_Self");
  return out;
}

}  // namespace
}  // namespace supa

TORCH_LIBRARY_IMPL(aten, PrivateUse1, m) {
  using namespace supa;
#define REG_UNARY(NAME)                      \
  m.impl(#NAME, TORCH_FN(pm_##NAME));        \
  m.impl(#NAME "_", TORCH_FN(pm_##NAME##_)); \
  m.impl(#NAME ".out", TORCH_FN(pm_##NAME##_out));
  REG_UNARY(sign)
  REG_UNARY(sgn)
  REG_UNARY(floor)
  REG_UNARY(ceil)
  REG_UNARY(round)
  REG_UNARY(trunc)
  REG_UNARY(rsqrt)
  REG_UNARY(bitwise_not)
  REG_UNARY(logical_not)
#undef REG_UNARY
#define REG_BITWISE(NAME)                                \
  m.impl(#NAME ".Tensor", TORCH_FN(NAME##_t));           \
  m.impl(#NAME "_.Tensor", TORCH_FN(NAME##_t_));         \
  m.impl(#NAME ".Tensor_out", TORCH_FN(NAME##_t_out));   \
  m.impl(#NAME ".Scalar", TORCH_FN(NAME##_s));           \
  m.impl(#NAME "_.Scalar", TORCH_FN(NAME##_s_));         \
  m.impl(#NAME ".Scalar_out", TORCH_FN(NAME##_s_out));
  REG_BITWISE(bitwise_and)
  REG_BITWISE(bitwise_or)
  REG_BITWISE(bitwise_xor)
#undef REG_BITWISE
#define REG_LOGICAL(NAME)                    \
  m.impl(#NAME, TORCH_FN(pm_##NAME));        \
  m.impl(#NAME "_", TORCH_FN(pm_##NAME##_)); \
  m.impl(#NAME ".out", TORCH_FN(pm_##NAME##_out));
  REG_LOGICAL(logical_and)
  REG_LOGICAL(logical_or)
  REG_LOGICAL(logical_xor)
#undef REG_LOGICAL
  m.impl("pow.Tensor_Scalar", TORCH_FN(pow_ts));
  m.impl("pow.Tensor_Scalar_out", TORCH_FN(pow_ts_out));
  m.impl("pow_.Scalar", TORCH_FN(pow_ts_));
  m.impl("pow.Tensor_Tensor", TORCH_FN(pow_tt));
  m.impl("pow.Tensor_Tensor_out", TORCH_FN(pow_tt_out));
  m.impl("pow_.Tensor", TORCH_FN(pow_tt_));
  m.impl("pow.Scalar", TORCH_FN(pow_st));
  m.impl("pow.Scalar_out", TORCH_FN(pow_st_out));
  m.impl("special_xlog1py", TORCH_FN(xlog1py_t));
  m.impl("special_xlog1py.out", TORCH_FN(xlog1py_t_out));
  m.impl("special_xlog1py.other_scalar", TORCH_FN(xlog1py_so));
  m.impl("special_xlog1py.other_scalar_out", TORCH_FN(xlog1py_so_out));
  m.impl("special_xlog1py.self_scalar", TORCH_FN(xlog1py_ss));
  m.impl("special_xlog1py.self_scalar_out", TORCH_FN(xlog1py_ss_out));
  m.impl("xlogy.Tensor", TORCH_FN(xlogy_t));
  m.impl("xlogy.OutTensor", TORCH_FN(xlogy_t_out));
  m.impl("xlogy_.Tensor", TORCH_FN(xlogy_t_));
  m.impl("xlogy.Scalar_Other", TORCH_FN(xlogy_so));
  m.impl("xlogy.OutScalar_Other", TORCH_FN(xlogy_so_out));
  m.impl("xlogy_.Scalar_Other", TORCH_FN(xlogy_so_));
  m.impl("xlogy.Scalar_Self", TORCH_FN(xlogy_ss));
  m.impl("xlogy.OutScalar_Self", TORCH_FN(xlogy_ss_out));
}
