// PrivateUse1 registrations of the optimizer path: the _foreach_* family
// (add / sub / mul / div / maximum / minimum / clamp_min / clamp_max in their
// List, Scalar, ScalarList and Tensor forms; addcmul / addcdiv; lerp; pow in
// its List, Scalar, ScalarList and ScalarAndTensor forms; the unary ops the
// elementwise kernels have; copy_; zero_; norm), in-place and
// out-of-place, _fused_adamw_, and the mixed-precision pieces beside it
// (_amp_foreach_non_finite_check_and_unscale_, _amp_update_scale_).
//
// Fast path: every tensor on one supa device, one floating dtype, dense and
// contiguous (and, across lists, matching shapes), real scalars -- then one
// multi-tensor-apply launch per 40 tensors.  Anything else takes the slow
// path the upstream CompositeExplicitAutograd foreach kernels take: one
// elementwise op per tensor (still on the supa kernels where they exist).
#include <ATen/WrapDimUtilsMulti.h>
#include <ATen/native/ForeachUtils.h>
#include <ATen/native/Resize.h>
#include <ATen/native/CPUFallback.h>
#include <ATen/ops/linalg_vector_norm.h>
#include <ATen/ops/linalg_vector_norm_ops.h>
#include <torch/library.h>

#include <bitset>
#include <cmath>
#include <map>

#include "common.h"

namespace supa {
namespace {

bool float_family(c10::ScalarType t) {
  return t == at::kFloat || t == at::kBFloat16 || t == at::kHalf || t == at::kDouble;
}

bool fast_ok(std::initializer_list<at::TensorList> lists) {
  c10::ScalarType dt = c10::ScalarType::Undefined;
  c10::Device dev(kSupa, 0);
  bool first = true;
  size_t n = 0;
  for (const auto& l : lists) {
    if (first) n = l.size();
    if (l.size() != n) return false;
    for (size_t i = 0; i < l.size(); ++i) {
      const at::Tensor& t = l[i];
      if (t.device().type() != kSupa || !t.is_contiguous() || !float_family(t.scalar_type())) return false;
      if (first && i == 0) {
        dt = t.scalar_type();
        dev = t.device();
      }
      if (t.scalar_type() != dt || t.device() != dev) return false;
      if (!first && t.sizes() != lists.begin()->at(i).sizes()) return false;
    }
    first = false;
  }
  return true;
}

// ------------------------------------------------------- generic launch
std::vector<at::Tensor> empty_like_list(at::TensorList a) {
  std::vector<at::Tensor> out;
  out.reserve(a.size());
  for (const auto& t : a) out.push_back(at::empty_like(t));
  return out;
}

// One supa_amd_foreach call over lists that passed fast_ok.
void fe_launch(int op, int form, at::TensorList out, at::TensorList a, at::TensorList b, at::TensorList c,
               const std::vector<double>& scalars, double alpha, const at::Tensor& dev_scalar, const char* name) {
  const size_t n = out.size();
  if (n == 0) return;
  std::vector<void*> po(n);
  std::vector<const void*> pa(a.size()), pb(b.size()), pc(c.size());
  std::vector<int64_t> numel(n);
  for (size_t i = 0; i < n; ++i) {
    po[i] = out[i].data_ptr();
    numel[i] = out[i].numel();
  }
  for (size_t i = 0; i < a.size(); ++i) pa[i] = a[i].data_ptr();
  for (size_t i = 0; i < b.size(); ++i) pb[i] = b[i].data_ptr();
  for (size_t i = 0; i < c.size(); ++i) pc[i] = c[i].data_ptr();
  const auto dev = out[0].device().index();
  const int rc = supa_amd_foreach(op, form, (int32_t)n, po.data(), a.empty() ? nullptr : pa.data(),
                                  b.empty() ? nullptr : pb.data(), c.empty() ? nullptr : pc.data(), numel.data(),
                                  dtype_code(out[0].scalar_type()), scalars.empty() ? nullptr : scalars.data(), alpha,
                                  dev_scalar.defined() ? dev_scalar.data_ptr() : nullptr, current_stream(dev));
  check_status(rc, name);
}

// A real (not complex, not bool) scalar: bool scalars keep upstream's
// per-tensor semantics through the slow path.
bool real_scalar(const c10::Scalar& s) { return !s.isComplex() && !s.isBoolean(); }
bool real_scalars(at::ArrayRef<c10::Scalar> ss) {
  for (const auto& s : ss)
    if (!real_scalar(s)) return false;
  return true;
}
std::vector<double> to_doubles(at::ArrayRef<c10::Scalar> ss) {
  std::vector<double> v;
  v.reserve(ss.size());
  for (const auto& s : ss) v.push_back(s.toDouble());
  return v;
}

// ------------------------------------------------------------- binary
// clamp_min is maximum and clamp_max is minimum (both NaN-propagating).
enum class Bop { Add, Sub, Mul, Div, Max, Min };

int bop_code(Bop o) {
  switch (o) {
    case Bop::Add:
    case Bop::Sub: return SUPA_AMD_FOREACH_ADD;
    case Bop::Mul: return SUPA_AMD_FOREACH_MUL;
    case Bop::Div: return SUPA_AMD_FOREACH_DIV;
    case Bop::Max: return SUPA_AMD_FOREACH_MAXIMUM;
    default: return SUPA_AMD_FOREACH_MINIMUM;
  }
}
const char* bop_name(Bop o) {
  static const char* names[] = {"_foreach_add", "_foreach_sub", "_foreach_mul", "_foreach_div", "_foreach_maximum",
                                "_foreach_minimum"};
  return names[(int)o];
}

// The slow path: the per-tensor op (upstream's CompositeExplicit foreach
// kernels do the same), with a tensor or a scalar second operand.
at::Tensor bop_one(Bop o, const at::Tensor& a, const at::Tensor& y, const c10::Scalar& alpha, bool inplace) {
  at::Tensor& s = const_cast<at::Tensor&>(a);
  switch (o) {
    case Bop::Add: return inplace ? s.add_(y, alpha) : at::add(a, y, alpha);
    case Bop::Sub: return inplace ? s.sub_(y, alpha) : at::sub(a, y, alpha);
    case Bop::Mul: return inplace ? s.mul_(y) : at::mul(a, y);
    case Bop::Div: return inplace ? s.div_(y) : at::div(a, y);
    case Bop::Max: return inplace ? s.clamp_min_(y) : at::clamp_min(a, y);
    default: return inplace ? s.clamp_max_(y) : at::clamp_max(a, y);
  }
}
at::Tensor bop_one(Bop o, const at::Tensor& a, const c10::Scalar& y, bool inplace) {
  at::Tensor& s = const_cast<at::Tensor&>(a);
  switch (o) {
    case Bop::Add: return inplace ? s.add_(y) : at::add(a, y);
    case Bop::Sub: return inplace ? s.sub_(y) : at::sub(a, y);
    case Bop::Mul: return inplace ? s.mul_(y) : at::mul(a, y);
    case Bop::Div: return inplace ? s.div_(y) : at::div(a, y);
    case Bop::Max: return inplace ? s.clamp_min_(y) : at::clamp_min(a, y);
    default: return inplace ? s.clamp_max_(y) : at::clamp_max(a, y);
  }
}

// List form: out[k] = a[k] op b[k] (add / sub with alpha).
std::vector<at::Tensor> bop_list(Bop o, at::TensorList self, at::TensorList other, const c10::Scalar& alpha,
                                 bool inplace) {
  at::native::check_foreach_api_restrictions(self, other);
  if (fast_ok({self, other}) && real_scalar(alpha)) {
    std::vector<at::Tensor> out = inplace ? self.vec() : empty_like_list(self);
    const double al = o == Bop::Sub ? -alpha.toDouble() : alpha.toDouble();
    fe_launch(bop_code(o), SUPA_AMD_FOREACH_LIST, out, self, other, {}, {}, al, {}, bop_name(o));
    return out;
  }
  std::vector<at::Tensor> out;
  for (size_t i = 0; i < self.size(); ++i) out.push_back(bop_one(o, self[i], other[i], alpha, inplace));
  return out;
}

// Scalar and ScalarList forms: out[k] = a[k] op s[k]; sub is add of -s.
std::vector<at::Tensor> bop_scalars(Bop o, at::TensorList self, at::ArrayRef<c10::Scalar> ss, bool inplace) {
  at::native::check_foreach_api_restrictions(self, ss);
  if (fast_ok({self}) && real_scalars(ss)) {
    std::vector<at::Tensor> out = inplace ? self.vec() : empty_like_list(self);
    std::vector<double> v = to_doubles(ss);
    if (o == Bop::Sub)
      for (double& x : v) x = -x;
    fe_launch(bop_code(o), SUPA_AMD_FOREACH_SCALARS, out, self, {}, {}, v, 1.0, {}, bop_name(o));
    return out;
  }
  std::vector<at::Tensor> out;
  for (size_t i = 0; i < self.size(); ++i) out.push_back(bop_one(o, self[i], ss[i], inplace));
  return out;
}
std::vector<at::Tensor> bop_scalar(Bop o, at::TensorList self, const c10::Scalar& s, bool inplace) {
  std::vector<c10::Scalar> ss(self.size(), s);
  at::native::check_foreach_api_restrictions(self);
  return bop_scalars(o, self, ss, inplace);
}

// Tensor form: a 0-dim tensor on the list's device is read by the kernel
// (after a cast to the list dtype, which is what the per-tensor op does with
// a 0-dim operand of the same category); elsewhere the per-tensor op.
std::vector<at::Tensor> bop_tensor(Bop o, at::TensorList self, const at::Tensor& other, const c10::Scalar& alpha,
                                   bool inplace) {
  at::native::check_foreach_api_restrictions(self);
  TORCH_CHECK(other.dim() == 0 && other.numel() == 1, "scalar tensor expected to be 0 dim but it has ", other.dim(),
              " dimensions and ", other.numel(), " elements.");
  if (fast_ok({self}) && other.device() == self[0].device() && float_family(other.scalar_type()) &&
      real_scalar(alpha)) {
    std::vector<at::Tensor> out = inplace ? self.vec() : empty_like_list(self);
    const at::Tensor y = other.scalar_type() == self[0].scalar_type() ? other : other.to(self[0].scalar_type());
    const double al = o == Bop::Sub ? -alpha.toDouble() : alpha.toDouble();
    fe_launch(bop_code(o), SUPA_AMD_FOREACH_DEVSCALAR, out, self, {}, {}, {}, al, y, bop_name(o));
    return out;
  }
  std::vector<at::Tensor> out;
  for (size_t i = 0; i < self.size(); ++i) out.push_back(bop_one(o, self[i], other, alpha, inplace));
  return out;
}

// ------------------------------------------------------------ ternary
std::vector<at::Tensor> addc(bool div, at::TensorList self, at::TensorList t1, at::TensorList t2,
                             at::ArrayRef<c10::Scalar> values, bool inplace) {
  at::native::check_foreach_api_restrictions(self, t1, t2, values);
  const char* name = div ? "_foreach_addcdiv" : "_foreach_addcmul";
  if (fast_ok({self, t1, t2}) && real_scalars(values)) {
    std::vector<at::Tensor> out = inplace ? self.vec() : empty_like_list(self);
    fe_launch(div ? SUPA_AMD_FOREACH_ADDCDIV : SUPA_AMD_FOREACH_ADDCMUL, SUPA_AMD_FOREACH_SCALARS, out, self, t1, t2,
              to_doubles(values), 1.0, {}, name);
    return out;
  }
  std::vector<at::Tensor> out;
  for (size_t i = 0; i < self.size(); ++i) {
    at::Tensor& s = const_cast<at::Tensor&>(self[i]);
    if (div) out.push_back(inplace ? s.addcdiv_(t1[i], t2[i], values[i]) : at::addcdiv(s, t1[i], t2[i], values[i]));
    else out.push_back(inplace ? s.addcmul_(t1[i], t2[i], values[i]) : at::addcmul(s, t1[i], t2[i], values[i]));
  }
  return out;
}

std::vector<at::Tensor> lerp_list(at::TensorList self, at::TensorList ends, at::TensorList weights, bool inplace) {
  at::native::check_foreach_api_restrictions(self, ends, weights);
  if (fast_ok({self, ends, weights})) {
    std::vector<at::Tensor> out = inplace ? self.vec() : empty_like_list(self);
    fe_launch(SUPA_AMD_FOREACH_LERP, SUPA_AMD_FOREACH_LIST, out, self, ends, weights, {}, 1.0, {}, "_foreach_lerp");
    return out;
  }
  std::vector<at::Tensor> out;
  for (size_t i = 0; i < self.size(); ++i) {
    at::Tensor& s = const_cast<at::Tensor&>(self[i]);
    out.push_back(inplace ? s.lerp_(ends[i], weights[i]) : at::lerp(s, ends[i], weights[i]));
  }
  return out;
}
std::vector<at::Tensor> lerp_scalars(at::TensorList self, at::TensorList ends, at::ArrayRef<c10::Scalar> w,
                                     bool inplace) {
  at::native::check_foreach_api_restrictions(self, ends, w);
  if (fast_ok({self, ends}) && real_scalars(w)) {
    std::vector<at::Tensor> out = inplace ? self.vec() : empty_like_list(self);
    fe_launch(SUPA_AMD_FOREACH_LERP, SUPA_AMD_FOREACH_SCALARS, out, self, ends, {}, to_doubles(w), 1.0, {},
              "_foreach_lerp");
    return out;
  }
  std::vector<at::Tensor> out;
  for (size_t i = 0; i < self.size(); ++i) {
    at::Tensor& s = const_cast<at::Tensor&>(self[i]);
    out.push_back(inplace ? s.lerp_(ends[i], w[i]) : at::lerp(s, ends[i], w[i]));
  }
  return out;
}

// -------------------------------------------------------------- unary
at::Tensor unary_one(int u, const at::Tensor& a, bool inplace) {
  at::Tensor& s = const_cast<at::Tensor&>(a);
  switch (u) {
    case SUPA_AMD_SIGMOID: return inplace ? s.sigmoid_() : at::sigmoid(a);
    case SUPA_AMD_TANH: return inplace ? s.tanh_() : at::tanh(a);
    case SUPA_AMD_EXP: return inplace ? s.exp_() : at::exp(a);
    case SUPA_AMD_LOG: return inplace ? s.log_() : at::log(a);
    case SUPA_AMD_ERF: return inplace ? s.erf_() : at::erf(a);
    case SUPA_AMD_NEG: return inplace ? s.neg_() : at::neg(a);
    case SUPA_AMD_RECIPROCAL: return inplace ? s.reciprocal_() : at::reciprocal(a);
    case SUPA_AMD_ABS: return inplace ? s.abs_() : at::abs(a);
    case SUPA_AMD_EXPM1: return inplace ? s.expm1_() : at::expm1(a);
    case SUPA_AMD_LOG1P: return inplace ? s.log1p_() : at::log1p(a);
    case SUPA_AMD_SIGN: return inplace ? s.sign_() : at::sign(a);
    case SUPA_AMD_FLOOR: return inplace ? s.floor_() : at::floor(a);
    case SUPA_AMD_CEIL: return inplace ? s.ceil_() : at::ceil(a);
    case SUPA_AMD_ROUND: return inplace ? s.round_() : at::round(a);
    case SUPA_AMD_TRUNC: return inplace ? s.trunc_() : at::trunc(a);
    case SUPA_AMD_RSQRT: return inplace ? s.rsqrt_() : at::rsqrt(a);
    default: return inplace ? s.sqrt_() : at::sqrt(a);
  }
}
std::vector<at::Tensor> unary(int u, at::TensorList self, bool inplace, const char* name) {
  at::native::check_foreach_api_restrictions(self);
  if (fast_ok({self})) {
    std::vector<at::Tensor> out = inplace ? self.vec() : empty_like_list(self);
    fe_launch(SUPA_AMD_FOREACH_UNARY + u, SUPA_AMD_FOREACH_SCALARS, out, self, {}, {}, {}, 1.0, {}, name);
    return out;
  }
  std::vector<at::Tensor> out;
  for (const auto& t : self) out.push_back(unary_one(u, t, inplace));
  return out;
}

// ---------------------------------------------------------------- pow
// The per-tensor pow(Tensor, Scalar) rounds the exponent to the tensor's
// dtype before choosing its special cases; the multi-tensor kernel takes
// exponents that round to themselves, the rest go tensor by tensor.
bool exact_in(c10::ScalarType dt, double e) {
  switch (dt) {
    case at::kDouble: return true;
    case at::kFloat: return (double)(float)e == e;
    case at::kBFloat16: return (double)(float)c10::BFloat16((float)e) == e;
    case at::kHalf: return (double)(float)c10::Half((float)e) == e;
    default: return false;
  }
}

at::Tensor pow_one(const at::Tensor& a, const c10::Scalar& e, bool inplace) {
  return inplace ? const_cast<at::Tensor&>(a).pow_(e) : at::pow(a, e);
}

std::vector<at::Tensor> pow_list(at::TensorList self, at::TensorList exps, bool inplace) {
  at::native::check_foreach_api_restrictions(self, exps);
  if (fast_ok({self, exps})) {
    std::vector<at::Tensor> out = inplace ? self.vec() : empty_like_list(self);
    fe_launch(SUPA_AMD_FOREACH_POW, SUPA_AMD_FOREACH_LIST, out, self, exps, {}, {}, 1.0, {}, "_foreach_pow");
    return out;
  }
  std::vector<at::Tensor> out;
  for (size_t i = 0; i < self.size(); ++i)
    out.push_back(inplace ? const_cast<at::Tensor&>(self[i]).pow_(exps[i]) : at::pow(self[i], exps[i]));
  return out;
}

std::vector<at::Tensor> pow_scalars(at::TensorList self, at::ArrayRef<c10::Scalar> es, bool inplace) {
  at::native::check_foreach_api_restrictions(self, es);
  bool fast = fast_ok({self}) && real_scalars(es);
  for (size_t i = 0; fast && i < es.size(); ++i) fast = exact_in(self[0].scalar_type(), es[i].toDouble());
  if (fast) {
    std::vector<at::Tensor> out = inplace ? self.vec() : empty_like_list(self);
    fe_launch(SUPA_AMD_FOREACH_POW, SUPA_AMD_FOREACH_SCALARS, out, self, {}, {}, to_doubles(es), 1.0, {},
              "_foreach_pow");
    return out;
  }
  std::vector<at::Tensor> out;
  for (size_t i = 0; i < self.size(); ++i) out.push_back(pow_one(self[i], es[i], inplace));
  return out;
}

void pow_list_(at::TensorList s, at::TensorList e) { pow_list(s, e, true); }
std::vector<at::Tensor> pow_list_f(at::TensorList s, at::TensorList e) { return pow_list(s, e, false); }
void pow_scalar_(at::TensorList s, const c10::Scalar& e) { pow_scalars(s, std::vector<c10::Scalar>(s.size(), e), true); }
std::vector<at::Tensor> pow_scalar(at::TensorList s, const c10::Scalar& e) {
  return pow_scalars(s, std::vector<c10::Scalar>(s.size(), e), false);
}
void pow_scalarlist_(at::TensorList s, at::ArrayRef<c10::Scalar> e) { pow_scalars(s, e, true); }
std::vector<at::Tensor> pow_scalarlist(at::TensorList s, at::ArrayRef<c10::Scalar> e) { return pow_scalars(s, e, false); }

// base ** exps[k]: the base is read in the list's opmath type, as the
// per-tensor pow(Scalar, Tensor) binds it; a base of 1 (ones, whatever the
// exponent) goes tensor by tensor.
std::vector<at::Tensor> pow_scalar_base(const c10::Scalar& base, at::TensorList exps) {
  at::native::check_foreach_api_restrictions(exps);
  if (fast_ok({exps}) && real_scalar(base) && !base.equal(1.0)) {
    std::vector<at::Tensor> out = empty_like_list(exps);
    fe_launch(SUPA_AMD_FOREACH_RPOW, SUPA_AMD_FOREACH_SCALARS, out, exps, {}, {},
              std::vector<double>(exps.size(), base.toDouble()), 1.0, {}, "_foreach_pow");
    return out;
  }
  std::vector<at::Tensor> out;
  for (const auto& t : exps) out.push_back(at::pow(base, t));
  return out;
}

// _foreach_copy_: same-dtype dense lists in one launch, otherwise copy_ per
// tensor (casts, layouts, other devices).
void foreach_copy_(at::TensorList self, at::TensorList src, bool non_blocking) {
  at::native::check_foreach_api_restrictions(self, src);
  if (fast_ok({self, src}))
    return fe_launch(SUPA_AMD_FOREACH_COPY, SUPA_AMD_FOREACH_SCALARS, self, src, {}, {}, {}, 1.0, {},
                     "_foreach_copy_");
  for (size_t i = 0; i < self.size(); ++i) const_cast<at::Tensor&>(self[i]).copy_(src[i], non_blocking);
}

void foreach_zero_(at::TensorList self) {
  if (fast_ok({self})) return fe_launch(SUPA_AMD_FOREACH_ZERO, SUPA_AMD_FOREACH_SCALARS, self, {}, {}, {}, {}, 1.0, {},
                                        "_foreach_zero_");
  for (const auto& t : self) const_cast<at::Tensor&>(t).zero_();
}

// --------------------------------------------------------------- norm
bool norm_ord_ok(const c10::Scalar& ord, double* p) {
  if (ord.isComplex()) return false;
  *p = ord.toDouble();
  return *p == 1.0 || *p == 2.0 || *p == HUGE_VAL;
}

// Norms of the listed (contiguous, one dtype) tensors into the n contiguous
// elements of `out`, in one pair of launches.
void norms_into(at::TensorList xs, double p, const at::Tensor& out, const char* name) {
  const size_t n = xs.size();
  std::vector<const void*> px(n);
  std::vector<int64_t> numel(n);
  for (size_t i = 0; i < n; ++i) {
    px[i] = xs[i].data_ptr();
    numel[i] = xs[i].numel();
  }
  const int32_t dt = dtype_code(xs[0].scalar_type());
  const int64_t ws_bytes = supa_amd_foreach_norm_workspace_bytes((int32_t)n, numel.data(), dt);
  TORCH_CHECK(ws_bytes >= 0, name, ": ", supa_amd_status_string((int)ws_bytes));
  at::Tensor ws = at::empty({std::max<int64_t>(ws_bytes, 1)}, xs[0].options().dtype(at::kByte));
  const int rc = supa_amd_foreach_norm((int32_t)n, px.data(), numel.data(), dt, p, out.data_ptr(),
                                       dtype_code(out.scalar_type()), ws.data_ptr(), ws_bytes,
                                       current_stream(xs[0].device().index()));
  check_status(rc, name);
}

// Per-tensor 1-, 2- and inf-norms; the results are views of one n-element
// tensor, as upstream's.  Other orders and dtypes take the per-tensor
// linalg_vector_norm.
std::vector<at::Tensor> foreach_norm(at::TensorList self, const c10::Scalar& ord, std::optional<at::ScalarType> dtype) {
  at::native::check_foreach_api_restrictions(self);
  double p = 0.0;
  const c10::ScalarType in_dt = self[0].scalar_type();
  const c10::ScalarType res_dt = dtype.value_or(in_dt);
  const bool fast = fast_ok({self}) && norm_ord_ok(ord, &p) &&
                    (res_dt == in_dt || res_dt == at::kFloat || res_dt == at::kDouble);
  std::vector<at::Tensor> res;
  if (!fast) {
    for (const auto& t : self) res.push_back(at::linalg_vector_norm(t, ord, at::OptionalIntArrayRef{}, false, dtype));
    return res;
  }
  at::Tensor out = at::empty({(int64_t)self.size()}, self[0].options().dtype(res_dt));
  norms_into(self, p, out, "_foreach_norm");
  res.reserve(self.size());
  for (size_t i = 0; i < self.size(); ++i) res.push_back(out.select(0, (int64_t)i));
  return res;
}

// linalg_vector_norm.  Over every element of a contiguous tensor with ord
// 1 / 2 / inf: the multi-tensor norm kernels with a one-tensor list.  Any
// other dims or order: the reduced dims go last in a contiguous copy and the
// row-norm kernel reduces each row.  A dtype of double on a narrower input
// converts the input first (upstream computes in the result dtype then);
// bf16 / f16 into f32 reads the narrow input directly.  Empty reductions
// without an identity (negative or infinite order) and complex inputs go to
// the CPU fallback, which raises or counts them.
at::Tensor vector_norm_supa(const at::Tensor& self, const c10::Scalar& ord, at::OptionalIntArrayRef dim,
                            bool keepdim, std::optional<at::ScalarType> dtype) {
  const c10::ScalarType in_dt = self.scalar_type();
  const c10::ScalarType res_dt = dtype.value_or(in_dt);
  const double p = ord.isComplex() ? NAN : ord.toDouble();
  const bool dt_ok = res_dt == in_dt || res_dt == at::kDouble || (res_dt == at::kFloat && in_dt != at::kDouble);
  const bool all_dims = !dim.has_value() || dim->empty();
  const int64_t nd = self.dim();
  std::bitset<at::dim_bitset_size> red;
  bool empty_reduction = false;
  if (all_dims) {
    for (int64_t i = 0; i < nd; ++i) red.set(i);
  } else {
    red = at::dim_list_to_bitset(*dim, nd);  // wraps, and rejects repeated dims
  }
  for (int64_t i = 0; i < nd; ++i) empty_reduction |= red[i] && self.size(i) == 0;
  if (self.device().type() != kSupa || !float_family(in_dt) || p != p || !dt_ok ||
      (empty_reduction && (p < 0 || std::isinf(p)))) {
    return at::native::call_fallback_fn<&supa_cpu_fallback, at::_ops::linalg_vector_norm>::call(self, ord, dim,
                                                                                             keepdim, dtype);
  }
  const at::Tensor x = (res_dt == at::kDouble && in_dt != at::kDouble) ? self.to(at::kDouble) : self;
  if (all_dims && x.is_contiguous() && (p == 1.0 || p == 2.0 || p == HUGE_VAL)) {
    std::vector<int64_t> shape(keepdim ? nd : 0, 1);
    at::Tensor out = at::empty(shape, x.options().dtype(res_dt));
    const at::Tensor list[1] = {x};
    norms_into(at::TensorList(list, 1), p, out, "linalg_vector_norm");
    return out;
  }
  std::vector<int64_t> oshape, perm;
  int64_t inner = 1, outer = 1;
  for (int64_t i = 0; i < nd; ++i) {
    if (!red[i]) {
      oshape.push_back(x.size(i));
      perm.push_back(i);
      outer *= x.size(i);
    } else if (keepdim) {
      oshape.push_back(1);
    }
  }
  for (int64_t i = 0; i < nd; ++i) {
    if (red[i]) {
      perm.push_back(i);
      inner *= x.size(i);
    }
  }
  at::Tensor out = at::empty(oshape, x.options().dtype(res_dt));
  if (outer == 0) return out;
  if (inner == 0) return out.zero_();  // an empty sum (orders >= 0)
  const at::Tensor rows = nd == 0 ? x.reshape({1}) : x.permute(perm).contiguous();
  const int32_t dt = dtype_code(x.scalar_type());
  const int64_t ws_bytes = supa_amd_norm_rows_workspace_bytes(outer, inner, dt);
  TORCH_CHECK(ws_bytes >= 0, "linalg_vector_norm: ", supa_amd_status_string((int)ws_bytes));
  at::Tensor ws;
  if (ws_bytes > 0) ws = at::empty({ws_bytes}, x.options().dtype(at::kByte));
  check_status(supa_amd_norm_rows(rows.data_ptr(), dt, out.data_ptr(), dtype_code(res_dt), outer, inner, p,
                                  ws_bytes > 0 ? ws.data_ptr() : nullptr, ws_bytes,
                                  current_stream(x.device().index())),
               "linalg_vector_norm");
  return out;
}

at::Tensor& vector_norm_out(const at::Tensor& self, const c10::Scalar& ord, at::OptionalIntArrayRef dim, bool keepdim,
                            std::optional<at::ScalarType> dtype, at::Tensor& out) {
  const at::Tensor r = vector_norm_supa(self, ord, dim, keepdim, dtype);
  TORCH_CHECK(out.scalar_type() == r.scalar_type(), "linalg.vector_norm: Expected out tensor to have dtype ",
              r.scalar_type(), ", but got ", out.scalar_type(), " instead");
  at::native::resize_output(out, r.sizes());
  out.copy_(r);
  return out;
}

// ------------------------------------------------ registered signatures
#define SUPA_FE_BINARY(NAME, OP)                                                                                    \
  void NAME##_list_(at::TensorList s, at::TensorList o) { bop_list(OP, s, o, 1, true); }                            \
  std::vector<at::Tensor> NAME##_list(at::TensorList s, at::TensorList o) { return bop_list(OP, s, o, 1, false); } \
  void NAME##_scalar_(at::TensorList s, const c10::Scalar& v) { bop_scalar(OP, s, v, true); }                       \
  std::vector<at::Tensor> NAME##_scalar(at::TensorList s, const c10::Scalar& v) { return bop_scalar(OP, s, v, false); } \
  void NAME##_scalarlist_(at::TensorList s, at::ArrayRef<c10::Scalar> v) { bop_scalars(OP, s, v, true); }          \
  std::vector<at::Tensor> NAME##_scalarlist(at::TensorList s, at::ArrayRef<c10::Scalar> v) {                        \
    return bop_scalars(OP, s, v, false);                                                                            \
  }
// add / sub take alpha in the List form
void add_list_(at::TensorList s, at::TensorList o, const c10::Scalar& a) { bop_list(Bop::Add, s, o, a, true); }
std::vector<at::Tensor> add_list(at::TensorList s, at::TensorList o, const c10::Scalar& a) {
  return bop_list(Bop::Add, s, o, a, false);
}
void sub_list_(at::TensorList s, at::TensorList o, const c10::Scalar& a) { bop_list(Bop::Sub, s, o, a, true); }
std::vector<at::Tensor> sub_list(at::TensorList s, at::TensorList o, const c10::Scalar& a) {
  return bop_list(Bop::Sub, s, o, a, false);
}
void add_scalar_(at::TensorList s, const c10::Scalar& v) { bop_scalar(Bop::Add, s, v, true); }
std::vector<at::Tensor> add_scalar(at::TensorList s, const c10::Scalar& v) { return bop_scalar(Bop::Add, s, v, false); }
void add_scalarlist_(at::TensorList s, at::ArrayRef<c10::Scalar> v) { bop_scalars(Bop::Add, s, v, true); }
std::vector<at::Tensor> add_scalarlist(at::TensorList s, at::ArrayRef<c10::Scalar> v) {
  return bop_scalars(Bop::Add, s, v, false);
}
void sub_scalar_(at::TensorList s, const c10::Scalar& v) { bop_scalar(Bop::Sub, s, v, true); }
std::vector<at::Tensor> sub_scalar(at::TensorList s, const c10::Scalar& v) { return bop_scalar(Bop::Sub, s, v, false); }
void sub_scalarlist_(at::TensorList s, at::ArrayRef<c10::Scalar> v) { bop_scalars(Bop::Sub, s, v, true); }
std::vector<at::Tensor> sub_scalarlist(at::TensorList s, at::ArrayRef<c10::Scalar> v) {
  return bop_scalars(Bop::Sub, s, v, false);
}
void add_tensor_(at::TensorList s, const at::Tensor& o, const c10::Scalar& a) { bop_tensor(Bop::Add, s, o, a, true); }
std::vector<at::Tensor> add_tensor(at::TensorList s, const at::Tensor& o, const c10::Scalar& a) {
  return bop_tensor(Bop::Add, s, o, a, false);
}
SUPA_FE_BINARY(mul, Bop::Mul)
SUPA_FE_BINARY(div, Bop::Div)
SUPA_FE_BINARY(maximum, Bop::Max)
SUPA_FE_BINARY(minimum, Bop::Min)
#undef SUPA_FE_BINARY
void mul_tensor_(at::TensorList s, const at::Tensor& o) { bop_tensor(Bop::Mul, s, o, 1, true); }
std::vector<at::Tensor> mul_tensor(at::TensorList s, const at::Tensor& o) { return bop_tensor(Bop::Mul, s, o, 1, false); }
void div_tensor_(at::TensorList s, const at::Tensor& o) { bop_tensor(Bop::Div, s, o, 1, true); }
std::vector<at::Tensor> div_tensor(at::TensorList s, const at::Tensor& o) { return bop_tensor(Bop::Div, s, o, 1, false); }

#define SUPA_FE_ADDC(NAME, DIV)                                                                                     \
  void NAME##_scalar_(at::TensorList s, at::TensorList a, at::TensorList b, const c10::Scalar& v) {                 \
    addc(DIV, s, a, b, std::vector<c10::Scalar>(s.size(), v), true);                                                \
  }                                                                                                                 \
  std::vector<at::Tensor> NAME##_scalar(at::TensorList s, at::TensorList a, at::TensorList b, const c10::Scalar& v) { \
    return addc(DIV, s, a, b, std::vector<c10::Scalar>(s.size(), v), false);                                        \
  }                                                                                                                 \
  void NAME##_scalarlist_(at::TensorList s, at::TensorList a, at::TensorList b, at::ArrayRef<c10::Scalar> v) {      \
    addc(DIV, s, a, b, v, true);                                                                                    \
  }                                                                                                                 \
  std::vector<at::Tensor> NAME##_scalarlist(at::TensorList s, at::TensorList a, at::TensorList b,                   \
                                            at::ArrayRef<c10::Scalar> v) {                                          \
    return addc(DIV, s, a, b, v, false);                                                                            \
  }                                                                                                                 \
  void NAME##_tensor_(at::TensorList s, at::TensorList a, at::TensorList b, const at::Tensor& v) {                  \
    addc(DIV, s, a, b, at::native::convert_tensor_to_scalar_list(v, s.size()), true);                               \
  }                                                                                                                 \
  std::vector<at::Tensor> NAME##_tensor(at::TensorList s, at::TensorList a, at::TensorList b, const at::Tensor& v) { \
    return addc(DIV, s, a, b, at::native::convert_tensor_to_scalar_list(v, s.size()), false);                       \
  }
SUPA_FE_ADDC(addcmul, false)
SUPA_FE_ADDC(addcdiv, true)
#undef SUPA_FE_ADDC

void lerp_list_(at::TensorList s, at::TensorList e, at::TensorList w) { lerp_list(s, e, w, true); }
std::vector<at::Tensor> lerp_list_f(at::TensorList s, at::TensorList e, at::TensorList w) {
  return lerp_list(s, e, w, false);
}
void lerp_scalar_(at::TensorList s, at::TensorList e, const c10::Scalar& w) {
  lerp_scalars(s, e, std::vector<c10::Scalar>(s.size(), w), true);
}
std::vector<at::Tensor> lerp_scalar(at::TensorList s, at::TensorList e, const c10::Scalar& w) {
  return lerp_scalars(s, e, std::vector<c10::Scalar>(s.size(), w), false);
}
void lerp_scalarlist_(at::TensorList s, at::TensorList e, at::ArrayRef<c10::Scalar> w) { lerp_scalars(s, e, w, true); }
std::vector<at::Tensor> lerp_scalarlist(at::TensorList s, at::TensorList e, at::ArrayRef<c10::Scalar> w) {
  return lerp_scalars(s, e, w, false);
}

#define SUPA_FE_UNARY(NAME, U)                                                                             \
  void fe_##NAME##_(at::TensorList s) { unary(U, s, true, "_foreach_" #NAME "_"); }                         \
  std::vector<at::Tensor> fe_##NAME(at::TensorList s) { return unary(U, s, false, "_foreach_" #NAME); }
SUPA_FE_UNARY(sigmoid, SUPA_AMD_SIGMOID)
SUPA_FE_UNARY(tanh, SUPA_AMD_TANH)
SUPA_FE_UNARY(exp, SUPA_AMD_EXP)
SUPA_FE_UNARY(log, SUPA_AMD_LOG)
SUPA_FE_UNARY(erf, SUPA_AMD_ERF)
SUPA_FE_UNARY(neg, SUPA_AMD_NEG)
SUPA_FE_UNARY(reciprocal, SUPA_AMD_RECIPROCAL)
SUPA_FE_UNARY(abs, SUPA_AMD_ABS)
SUPA_FE_UNARY(sqrt, SUPA_AMD_SQRT)
SUPA_FE_UNARY(expm1, SUPA_AMD_EXPM1)
SUPA_FE_UNARY(log1p, SUPA_AMD_LOG1P)
SUPA_FE_UNARY(sign, SUPA_AMD_SIGN)
SUPA_FE_UNARY(floor, SUPA_AMD_FLOOR)
SUPA_FE_UNARY(ceil, SUPA_AMD_CEIL)
SUPA_FE_UNARY(round, SUPA_AMD_ROUND)
SUPA_FE_UNARY(trunc, SUPA_AMD_TRUNC)
SUPA_FE_UNARY(rsqrt, SUPA_AMD_RSQRT)
#undef SUPA_FE_UNARY

// ------------------------------------------------------------ fused AdamW
void fused_adamw_impl(at::TensorList params, at::TensorList grads, at::TensorList exp_avgs,
                      at::TensorList exp_avg_sqs, at::TensorList max_exp_avg_sqs, at::TensorList state_steps,
                      double lr, const at::Tensor& lr_tensor, double beta1, double beta2, double weight_decay,
                      double eps, bool amsgrad, bool maximize, const std::optional<at::Tensor>& grad_scale,
                      const std::optional<at::Tensor>& found_inf, bool l2 = false) {
  const size_t n = params.size();
  TORCH_CHECK(grads.size() == n && exp_avgs.size() == n && exp_avg_sqs.size() == n && state_steps.size() == n,
              "_fused_adamw_: tensor lists must have the same length");
  TORCH_CHECK(!amsgrad || max_exp_avg_sqs.size() == n, "_fused_adamw_: max_exp_avg_sqs must match params for amsgrad");
  if (n == 0) return;
  const auto dev = params[0].device();
  const c10::ScalarType dt = params[0].scalar_type();
  TORCH_CHECK(float_family(dt), "_fused_adamw_: unsupported dtype ", dt);
  std::vector<void*> p(n), g(n), m(n), v(n), vm(amsgrad ? n : 0), st(n);
  std::vector<int64_t> numel(n);
  for (size_t i = 0; i < n; ++i) {
    for (const at::Tensor* t : {&params[i], &grads[i], &exp_avgs[i], &exp_avg_sqs[i]}) {
      TORCH_CHECK(t->device() == dev && t->scalar_type() == dt && t->is_contiguous(),
                  "_fused_adamw_: params, grads and states must be contiguous ", dt, " tensors on ", dev);
      TORCH_CHECK(t->numel() == params[i].numel(), "_fused_adamw_: tensor sizes differ at index ", i);
    }
    TORCH_CHECK(state_steps[i].device() == dev && state_steps[i].scalar_type() == at::kFloat &&
                    state_steps[i].numel() == 1,
                "_fused_adamw_: each state_step must be a one-element float32 tensor on ", dev);
    p[i] = params[i].data_ptr();
    g[i] = grads[i].data_ptr();
    m[i] = exp_avgs[i].data_ptr();
    v[i] = exp_avg_sqs[i].data_ptr();
    st[i] = state_steps[i].data_ptr();
    if (amsgrad) {
      TORCH_CHECK(max_exp_avg_sqs[i].device() == dev && max_exp_avg_sqs[i].scalar_type() == dt &&
                      max_exp_avg_sqs[i].is_contiguous(),
                  "_fused_adamw_: max_exp_avg_sqs must match params");
      vm[i] = max_exp_avg_sqs[i].data_ptr();
    }
    numel[i] = params[i].numel();
  }
  const float* lr_ptr = nullptr;
  at::Tensor lr_f;
  if (lr_tensor.defined()) {
    if (lr_tensor.device().type() == kSupa) {
      lr_f = lr_tensor.to(at::kFloat);
      lr_ptr = lr_f.data_ptr<float>();
    } else {
      lr = lr_tensor.item<double>();
    }
  }
  at::Tensor gs, fi;
  if (grad_scale.has_value() && grad_scale->defined()) {
    gs = grad_scale->to(dev).to(at::kFloat);
  }
  if (found_inf.has_value() && found_inf->defined()) {
    fi = found_inf->to(dev).to(at::kFloat);
  }
  const auto entry = l2 ? supa_amd_fused_adam : supa_amd_fused_adamw;
  const int rc = entry(
      (int32_t)n, p.data(), g.data(), m.data(), v.data(), amsgrad ? vm.data() : nullptr, st.data(), numel.data(),
      dtype_code(dt), lr, lr_ptr, beta1, beta2, weight_decay, eps, amsgrad ? 1 : 0, maximize ? 1 : 0,
      gs.defined() ? gs.data_ptr<float>() : nullptr, fi.defined() ? fi.data_ptr<float>() : nullptr,
      current_stream(dev.index()));
  check_status(rc, l2 ? "_fused_adam_" : "_fused_adamw_");
}

void fused_adamw_(at::TensorList params, at::TensorList grads, at::TensorList exp_avgs, at::TensorList exp_avg_sqs,
                  at::TensorList max_exp_avg_sqs, at::TensorList state_steps, double lr, double beta1, double beta2,
                  double weight_decay, double eps, bool amsgrad, bool maximize,
                  const std::optional<at::Tensor>& grad_scale, const std::optional<at::Tensor>& found_inf) {
  fused_adamw_impl(params, grads, exp_avgs, exp_avg_sqs, max_exp_avg_sqs, state_steps, lr, at::Tensor(), beta1,
                   beta2, weight_decay, eps, amsgrad, maximize, grad_scale, found_inf);
}

// ------------------------------------------------------------- fused SGD
// upstream _fused_sgd_kernel_cuda_'s checks: a momentum buffer list exactly
// when momentum > 0; one device and dtype, contiguous tensors.
void fused_sgd_impl(at::TensorList params, at::TensorList grads, at::TensorList bufs, double weight_decay,
                    double momentum, double lr, const at::Tensor& lr_tensor, double dampening, bool nesterov,
                    bool maximize, bool is_first_step, const std::optional<at::Tensor>& grad_scale,
                    const std::optional<at::Tensor>& found_inf) {
  const size_t n = params.size();
  TORCH_CHECK(grads.size() == n, "_fused_sgd_: params and grads must have the same length");
  const bool mom = !bufs.empty();
  if (mom) {
    TORCH_CHECK(momentum > 0, "_fused_sgd_: expected momentum > 0 with a momentum buffer list, got ", momentum);
    TORCH_CHECK(bufs.size() == n, "_fused_sgd_: momentum_buffer_list must match params");
  } else {
    TORCH_CHECK(momentum == 0, "_fused_sgd_: expected momentum == 0 without a momentum buffer list, got ",
                momentum);
    if (is_first_step) TORCH_WARN_ONCE("`is_first_step` argument has no effect when `momentum_buffer_list` is empty");
  }
  if (n == 0) return;
  const auto dev = params[0].device();
  const c10::ScalarType dt = params[0].scalar_type();
  TORCH_CHECK(float_family(dt), "_fused_sgd_: unsupported dtype ", dt);
  std::vector<void*> p(n), g(n), b(mom ? n : 0);
  std::vector<int64_t> numel(n);
  for (size_t i = 0; i < n; ++i) {
    std::vector<const at::Tensor*> ts{&params[i], &grads[i]};
    if (mom) ts.push_back(&bufs[i]);
    for (const at::Tensor* t : ts) {
      TORCH_CHECK(t->device() == dev && t->scalar_type() == dt && t->is_contiguous(),
                  "_fused_sgd_: params, grads and momentum buffers must be contiguous ", dt, " tensors on ", dev);
      TORCH_CHECK(t->numel() == params[i].numel(), "_fused_sgd_: tensor sizes differ at index ", i);
    }
    p[i] = params[i].data_ptr();
    g[i] = grads[i].data_ptr();
    if (mom) b[i] = bufs[i].data_ptr();
    numel[i] = params[i].numel();
  }
  const float* lr_ptr = nullptr;
  at::Tensor lr_f;
  if (lr_tensor.defined()) {
    if (lr_tensor.device().type() == kSupa) {
      lr_f = lr_tensor.to(at::kFloat);
      lr_ptr = lr_f.data_ptr<float>();
    } else {
      lr = lr_tensor.item<double>();
    }
  }
  at::Tensor gs, fi;
  if (grad_scale.has_value() && grad_scale->defined()) gs = grad_scale->to(dev).to(at::kFloat);
  if (found_inf.has_value() && found_inf->defined()) fi = found_inf->to(dev).to(at::kFloat);
  const int rc = supa_amd_fused_sgd((int32_t)n, p.data(), g.data(), mom ? b.data() : nullptr, numel.data(),
                                    dtype_code(dt), weight_decay, momentum, lr, lr_ptr, dampening, nesterov ? 1 : 0,
                                    maximize ? 1 : 0, is_first_step ? 1 : 0,
                                    gs.defined() ? gs.data_ptr<float>() : nullptr,
                                    fi.defined() ? fi.data_ptr<float>() : nullptr, current_stream(dev.index()));
  check_status(rc, "_fused_sgd_");
}
void fused_sgd_(at::TensorList params, at::TensorList grads, at::TensorList bufs, double weight_decay,
                double momentum, double lr, double dampening, bool nesterov, bool maximize, bool is_first_step,
                const std::optional<at::Tensor>& grad_scale, const std::optional<at::Tensor>& found_inf) {
  fused_sgd_impl(params, grads, bufs, weight_decay, momentum, lr, at::Tensor(), dampening, nesterov, maximize,
                 is_first_step, grad_scale, found_inf);
}
void fused_sgd_tensor_lr_(at::TensorList params, at::TensorList grads, at::TensorList bufs, double weight_decay,
                          double momentum, const at::Tensor& lr, double dampening, bool nesterov, bool maximize,
                          bool is_first_step, const std::optional<at::Tensor>& grad_scale,
                          const std::optional<at::Tensor>& found_inf) {
  fused_sgd_impl(params, grads, bufs, weight_decay, momentum, 0.0, lr, dampening, nesterov, maximize, is_first_step,
                 grad_scale, found_inf);
}

// _fused_adam_: the same kernel in Adam mode (weight decay on the gradient)
void fused_adam_(at::TensorList params, at::TensorList grads, at::TensorList exp_avgs, at::TensorList exp_avg_sqs,
                 at::TensorList max_exp_avg_sqs, at::TensorList state_steps, double lr, double beta1, double beta2,
                 double weight_decay, double eps, bool amsgrad, bool maximize,
                 const std::optional<at::Tensor>& grad_scale, const std::optional<at::Tensor>& found_inf) {
  fused_adamw_impl(params, grads, exp_avgs, exp_avg_sqs, max_exp_avg_sqs, state_steps, lr, at::Tensor(), beta1,
                   beta2, weight_decay, eps, amsgrad, maximize, grad_scale, found_inf, true);
}
void fused_adam_tensor_lr_(at::TensorList params, at::TensorList grads, at::TensorList exp_avgs,
                           at::TensorList exp_avg_sqs, at::TensorList max_exp_avg_sqs, at::TensorList state_steps,
                           const at::Tensor& lr, double beta1, double beta2, double weight_decay, double eps,
                           bool amsgrad, bool maximize, const std::optional<at::Tensor>& grad_scale,
                           const std::optional<at::Tensor>& found_inf) {
  fused_adamw_impl(params, grads, exp_avgs, exp_avg_sqs, max_exp_avg_sqs, state_steps, 0.0, lr, beta1, beta2,
                   weight_decay, eps, amsgrad, maximize, grad_scale, found_inf, true);
}

void fused_adamw_tensor_lr_(at::TensorList params, at::TensorList grads, at::TensorList exp_avgs,
                            at::TensorList exp_avg_sqs, at::TensorList max_exp_avg_sqs, at::TensorList state_steps,
                            const at::Tensor& lr, double beta1, double beta2, double weight_decay, double eps,
                            bool amsgrad, bool maximize, const std::optional<at::Tensor>& grad_scale,
                            const std::optional<at::Tensor>& found_inf) {
  fused_adamw_impl(params, grads, exp_avgs, exp_avg_sqs, max_exp_avg_sqs, state_steps, 0.0, lr, beta1, beta2,
                   weight_decay, eps, amsgrad, maximize, grad_scale, found_inf);
}

// ------------------------------------------------------------- AMP
// _amp_foreach_non_finite_check_and_unscale_: one multi-tensor launch per
// dtype group of contiguous supa tensors; anything else (non-contiguous
// tensors) is unscaled tensor by tensor through the same kernel on a
// contiguous copy.
void amp_unscale_(at::TensorList self, at::Tensor& found_inf, const at::Tensor& inv_scale) {
  TORCH_CHECK(found_inf.numel() == 1 && found_inf.scalar_type() == at::kFloat && found_inf.device().type() == kSupa,
              "found_inf must be a one-element float tensor on the supa device");
  TORCH_CHECK(inv_scale.numel() == 1 && inv_scale.scalar_type() == at::kFloat && inv_scale.device().type() == kSupa,
              "inv_scale must be a one-element float tensor on the supa device");
  if (self.empty()) return;
  const auto dev = found_inf.device().index();
  std::map<c10::ScalarType, std::vector<at::Tensor>> groups;
  for (const at::Tensor& t : self) {
    TORCH_CHECK(t.device() == found_inf.device(), "_amp_foreach_non_finite_check_and_unscale_: tensors on ",
                t.device(), " and ", found_inf.device());
    TORCH_CHECK(float_family(t.scalar_type()), "_amp_foreach_non_finite_check_and_unscale_: expected floating "
                "tensors, got ", t.scalar_type());
    groups[t.scalar_type()].push_back(t);
  }
  for (auto& [dt, ts] : groups) {
    std::vector<at::Tensor> work, back;
    std::vector<void*> ptrs;
    std::vector<int64_t> numel;
    for (const at::Tensor& t : ts) {
      at::Tensor w = t.is_contiguous() ? t : t.contiguous();
      ptrs.push_back(w.data_ptr());
      numel.push_back(w.numel());
      work.push_back(w);
    }
    const int rc = supa_amd_amp_unscale((int32_t)ptrs.size(), ptrs.data(), numel.data(), dtype_code(dt),
                                        found_inf.data_ptr<float>(), inv_scale.data_ptr<float>(), current_stream(dev));
    check_status(rc, "_amp_foreach_non_finite_check_and_unscale_");
    for (size_t i = 0; i < ts.size(); ++i)
      if (!work[i].is_same(ts[i])) ts[i].copy_(work[i]);
  }
}

at::Tensor& amp_update_scale_(at::Tensor& self, at::Tensor& growth_tracker, const at::Tensor& found_inf,
                              double growth_factor, double backoff_factor, int64_t growth_interval) {
  TORCH_CHECK(self.numel() == 1 && self.scalar_type() == at::kFloat, "_amp_update_scale_: scale must be a "
              "one-element float tensor");
  TORCH_CHECK(growth_tracker.numel() == 1 && growth_tracker.scalar_type() == at::kInt,
              "_amp_update_scale_: growth_tracker must be a one-element int tensor");
  TORCH_CHECK(found_inf.numel() == 1 && found_inf.scalar_type() == at::kFloat,
              "_amp_update_scale_: found_inf must be a one-element float tensor");
  const auto dev = self.device().index();
  const int rc = supa_amd_amp_update_scale(self.data_ptr<float>(), growth_tracker.data_ptr<int32_t>(),
                                           found_inf.data_ptr<float>(), growth_factor, backoff_factor,
                                           growth_interval, current_stream(dev));
  check_status(rc, "_amp_update_scale_");
  return self;
}

}  // namespace
}  // namespace supa

TORCH_LIBRARY_IMPL(aten, PrivateUse1, m) {
  using namespace supa;
  // binary: List / Scalar / ScalarList / Tensor
  m.impl("_foreach_add_.List", TORCH_FN(add_list_));
  m.impl("_foreach_add.List", TORCH_FN(add_list));
  m.impl("_foreach_add_.Scalar", TORCH_FN(add_scalar_));
  m.impl("_foreach_add.Scalar", TORCH_FN(add_scalar));
  m.impl("_foreach_add_.ScalarList", TORCH_FN(add_scalarlist_));
  m.impl("_foreach_add.ScalarList", TORCH_FN(add_scalarlist));
  m.impl("_foreach_add_.Tensor", TORCH_FN(add_tensor_));
  m.impl("_foreach_add.Tensor", TORCH_FN(add_tensor));
  m.impl("_foreach_sub_.List", TORCH_FN(sub_list_));
  m.impl("_foreach_sub.List", TORCH_FN(sub_list));
  m.impl("_foreach_sub_.Scalar", TORCH_FN(sub_scalar_));
  m.impl("_foreach_sub.Scalar", TORCH_FN(sub_scalar));
  m.impl("_foreach_sub_.ScalarList", TORCH_FN(sub_scalarlist_));
  m.impl("_foreach_sub.ScalarList", TORCH_FN(sub_scalarlist));
#define SUPA_FE_REG_BINARY(SCHEMA, NAME)                                 \
  m.impl("_foreach_" SCHEMA "_.List", TORCH_FN(NAME##_list_));             \
  m.impl("_foreach_" SCHEMA ".List", TORCH_FN(NAME##_list));               \
  m.impl("_foreach_" SCHEMA "_.Scalar", TORCH_FN(NAME##_scalar_));         \
  m.impl("_foreach_" SCHEMA ".Scalar", TORCH_FN(NAME##_scalar));           \
  m.impl("_foreach_" SCHEMA "_.ScalarList", TORCH_FN(NAME##_scalarlist_)); \
  m.impl("_foreach_" SCHEMA ".ScalarList", TORCH_FN(NAME##_scalarlist));
  SUPA_FE_REG_BINARY("mul", mul)
  SUPA_FE_REG_BINARY("div", div)
  SUPA_FE_REG_BINARY("maximum", maximum)
  SUPA_FE_REG_BINARY("minimum", minimum)
  SUPA_FE_REG_BINARY("clamp_min", maximum)
  SUPA_FE_REG_BINARY("clamp_max", minimum)
#undef SUPA_FE_REG_BINARY
  m.impl("_foreach_mul_.Tensor", TORCH_FN(mul_tensor_));
  m.impl("_foreach_mul.Tensor", TORCH_FN(mul_tensor));
  m.impl("_foreach_div_.Tensor", TORCH_FN(div_tensor_));
  m.impl("_foreach_div.Tensor", TORCH_FN(div_tensor));
  // pointwise ternary
#define SUPA_FE_REG_ADDC(NAME)                                                \
  m.impl("_foreach_" #NAME "_.Scalar", TORCH_FN(NAME##_scalar_));             \
  m.impl("_foreach_" #NAME ".Scalar", TORCH_FN(NAME##_scalar));               \
  m.impl("_foreach_" #NAME "_.ScalarList", TORCH_FN(NAME##_scalarlist_));     \
  m.impl("_foreach_" #NAME ".ScalarList", TORCH_FN(NAME##_scalarlist));       \
  m.impl("_foreach_" #NAME "_.Tensor", TORCH_FN(NAME##_tensor_));             \
  m.impl("_foreach_" #NAME ".Tensor", TORCH_FN(NAME##_tensor));
  SUPA_FE_REG_ADDC(addcmul)
  SUPA_FE_REG_ADDC(addcdiv)
#undef SUPA_FE_REG_ADDC
  m.impl("_foreach_lerp_.List", TORCH_FN(lerp_list_));
  m.impl("_foreach_lerp.List", TORCH_FN(lerp_list_f));
  m.impl("_foreach_lerp_.Scalar", TORCH_FN(lerp_scalar_));
  m.impl("_foreach_lerp.Scalar", TORCH_FN(lerp_scalar));
  m.impl("_foreach_lerp_.ScalarList", TORCH_FN(lerp_scalarlist_));
  m.impl("_foreach_lerp.ScalarList", TORCH_FN(lerp_scalarlist));
  // unary, zero_, norm
#define SUPA_FE_REG_UNARY(NAME)                             \
  m.impl("_foreach_" #NAME "_", TORCH_FN(fe_##NAME##_));   \
  m.impl("_foreach_" #NAME, TORCH_FN(fe_##NAME));
  SUPA_FE_REG_UNARY(sigmoid)
  SUPA_FE_REG_UNARY(tanh)
  SUPA_FE_REG_UNARY(exp)
  SUPA_FE_REG_UNARY(log)
  SUPA_FE_REG_UNARY(erf)
  SUPA_FE_REG_UNARY(neg)
  SUPA_FE_REG_UNARY(reciprocal)
  SUPA_FE_REG_UNARY(abs)
  SUPA_FE_REG_UNARY(sqrt)
  SUPA_FE_REG_UNARY(expm1)
  SUPA_FE_REG_UNARY(log1p)
  SUPA_FE_REG_UNARY(sign)
  SUPA_FE_REG_UNARY(floor)
  SUPA_FE_REG_UNARY(ceil)
  SUPA_FE_REG_UNARY(round)
  SUPA_FE_REG_UNARY(trunc)
  SUPA_FE_REG_UNARY(rsqrt)
#undef SUPA_FE_REG_UNARY
  // pow, copy_
  m.impl("_foreach_pow_.List", TORCH_FN(pow_list_));
  m.impl("_foreach_pow.List", TORCH_FN(pow_list_f));
  m.impl("_foreach_pow_.Scalar", TORCH_FN(pow_scalar_));
  m.impl("_foreach_pow.Scalar", TORCH_FN(pow_scalar));
  m.impl("_foreach_pow_.ScalarList", TORCH_FN(pow_scalarlist_));
  m.impl("_foreach_pow.ScalarList", TORCH_FN(pow_scalarlist));
  m.impl("_foreach_pow.ScalarAndTensor", TORCH_FN(pow_scalar_base));
  m.impl("_foreach_copy_", TORCH_FN(foreach_copy_));
  m.impl("_foreach_zero_", TORCH_FN(foreach_zero_));
  m.impl("_foreach_norm.Scalar", TORCH_FN(foreach_norm));
  m.impl("linalg_vector_norm", TORCH_FN(vector_norm_supa));
  m.impl("linalg_vector_norm.out", TORCH_FN(vector_norm_out));
  m.impl("_fused_adamw_", TORCH_FN(fused_adamw_));
  m.impl("_fused_adamw_.tensor_lr", TORCH_FN(fused_adamw_tensor_lr_));
  m.impl("_fused_adam_", TORCH_FN(fused_adam_));
  m.impl("_fused_adam_.tensor_lr", TORCH_FN(fused_adam_tensor_lr_));
  m.impl("_fused_sgd_", TORCH_FN(fused_sgd_));
  m.impl("_fused_sgd_.tensor_lr", TORCH_FN(fused_sgd_tensor_lr_));
  m.impl("_amp_foreach_non_finite_check_and_unscale_", TORCH_FN(amp_unscale_));
  m.impl("_amp_update_scale_", TORCH_FN(amp_update_scale_));
}
