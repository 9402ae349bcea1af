// PrivateUse1 registrations of the optimizer path: _foreach_add / _foreach_mul
// (List and Scalar overloads, in-place and out-of-place), _fused_adamw_, and
// the mixed-precision pieces beside it (_amp_foreach_non_finite_check_and_unscale_,
// _amp_update_scale_).
//
// Fast path: every tensor on one supa device, one floating dtype, dense and
// contiguous (and, for List overloads, matching shapes) -- then one
// multi-tensor-apply launch per 40 tensors.  Anything else takes the slow
// path the upstream CompositeExplicitAutograd foreach kernels take: one
// elementwise op per tensor (still on the supa kernels).
#include <ATen/native/ForeachUtils.h>
#include <torch/library.h>

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

void launch_foreach(int op, at::TensorList out, at::TensorList a, at::TensorList b, double scalar, double alpha) {
  const size_t n = a.size();
  if (n == 0) return;
  std::vector<void*> po(n), pa(n), pb(b.empty() ? 0 : n);
  std::vector<int64_t> numel(n);
  for (size_t i = 0; i < n; ++i) {
    po[i] = out[i].data_ptr();
    pa[i] = a[i].data_ptr();
    if (!b.empty()) pb[i] = b[i].data_ptr();
    numel[i] = a[i].numel();
  }
  const auto dev = a[0].device().index();
  const int rc = supa_amd_foreach_binary(op, (int32_t)n, po.data(), pa.data(), b.empty() ? nullptr : pb.data(),
                                         numel.data(), dtype_code(a[0].scalar_type()), scalar, alpha,
                                         current_stream(dev));
  check_status(rc, op == SUPA_AMD_FOREACH_ADD ? "_foreach_add" : "_foreach_mul");
}

double scalar_value(const c10::Scalar& s) {
  TORCH_CHECK(!s.isComplex(), "supa foreach: complex scalars are not supported");
  return s.toDouble();
}

// ------------------------------------------------------------- add / mul
void foreach_add_scalar_(at::TensorList self, const c10::Scalar& s) {
  if (fast_ok({self}) && !s.isBoolean()) return launch_foreach(SUPA_AMD_FOREACH_ADD, self, self, {}, scalar_value(s), 1.0);
  for (const auto& t : self) const_cast<at::Tensor&>(t).add_(s);
}
std::vector<at::Tensor> foreach_add_scalar(at::TensorList self, const c10::Scalar& s) {
  if (fast_ok({self}) && !s.isBoolean()) {
    std::vector<at::Tensor> out;
    for (const auto& t : self) out.push_back(at::empty_like(t));
    launch_foreach(SUPA_AMD_FOREACH_ADD, out, self, {}, scalar_value(s), 1.0);
    return out;
  }
  std::vector<at::Tensor> out;
  for (const auto& t : self) out.push_back(t.add(s));
  return out;
}
void foreach_add_list_(at::TensorList self, at::TensorList other, const c10::Scalar& alpha) {
  at::native::check_foreach_api_restrictions(self, other);
  if (fast_ok({self, other})) return launch_foreach(SUPA_AMD_FOREACH_ADD, self, self, other, 0.0, scalar_value(alpha));
  for (size_t i = 0; i < self.size(); ++i) const_cast<at::Tensor&>(self[i]).add_(other[i], alpha);
}
std::vector<at::Tensor> foreach_add_list(at::TensorList self, at::TensorList other, const c10::Scalar& alpha) {
  at::native::check_foreach_api_restrictions(self, other);
  std::vector<at::Tensor> out;
  if (fast_ok({self, other})) {
    for (const auto& t : self) out.push_back(at::empty_like(t));
    launch_foreach(SUPA_AMD_FOREACH_ADD, out, self, other, 0.0, scalar_value(alpha));
    return out;
  }
  for (size_t i = 0; i < self.size(); ++i) out.push_back(self[i].add(other[i], alpha));
  return out;
}
void foreach_mul_scalar_(at::TensorList self, const c10::Scalar& s) {
  if (fast_ok({self}) && !s.isBoolean()) return launch_foreach(SUPA_AMD_FOREACH_MUL, self, self, {}, scalar_value(s), 1.0);
  for (const auto& t : self) const_cast<at::Tensor&>(t).mul_(s);
}
std::vector<at::Tensor> foreach_mul_scalar(at::TensorList self, const c10::Scalar& s) {
  std::vector<at::Tensor> out;
  if (fast_ok({self}) && !s.isBoolean()) {
    for (const auto& t : self) out.push_back(at::empty_like(t));
    launch_foreach(SUPA_AMD_FOREACH_MUL, out, self, {}, scalar_value(s), 1.0);
    return out;
  }
  for (const auto& t : self) out.push_back(t.mul(s));
  return out;
}
void foreach_mul_list_(at::TensorList self, at::TensorList other) {
  at::native::check_foreach_api_restrictions(self, other);
  if (fast_ok({self, other})) return launch_foreach(SUPA_AMD_FOREACH_MUL, self, self, other, 0.0, 1.0);
  for (size_t i = 0; i < self.size(); ++i) const_cast<at::Tensor&>(self[i]).mul_(other[i]);
}
std::vector<at::Tensor> foreach_mul_list(at::TensorList self, at::TensorList other) {
  at::native::check_foreach_api_restrictions(self, other);
  std::vector<at::Tensor> out;
  if (fast_ok({self, other})) {
    for (const auto& t : self) out.push_back(at::empty_like(t));
    launch_foreach(SUPA_AMD_FOREACH_MUL, out, self, other, 0.0, 1.0);
    return out;
  }
  for (size_t i = 0; i < self.size(); ++i) out.push_back(self[i].mul(other[i]));
  return out;
}

// ------------------------------------------------------------ fused AdamW
void fused_adamw_impl(at::TensorList params, at::TensorList grads, at::TensorList exp_avgs,
                      at::TensorList exp_avg_sqs, at::TensorList max_exp_avg_sqs, at::TensorList state_steps,
                      double lr, const at::Tensor& lr_tensor, double beta1, double beta2, double weight_decay,
                      double eps, bool amsgrad, bool maximize, const std::optional<at::Tensor>& grad_scale,
                      const std::optional<at::Tensor>& found_inf) {
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
  const int rc = supa_amd_fused_adamw(
      (int32_t)n, p.data(), g.data(), m.data(), v.data(), amsgrad ? vm.data() : nullptr, st.data(), numel.data(),
      dtype_code(dt), lr, lr_ptr, beta1, beta2, weight_decay, eps, amsgrad ? 1 : 0, maximize ? 1 : 0,
      gs.defined() ? gs.data_ptr<float>() : nullptr, fi.defined() ? fi.data_ptr<float>() : nullptr,
      current_stream(dev.index()));
  check_status(rc, "_fused_adamw_");
}

void fused_adamw_(at::TensorList params, at::TensorList grads, at::TensorList exp_avgs, at::TensorList exp_avg_sqs,
                  at::TensorList max_exp_avg_sqs, at::TensorList state_steps, double lr, double beta1, double beta2,
                  double weight_decay, double eps, bool amsgrad, bool maximize,
                  const std::optional<at::Tensor>& grad_scale, const std::optional<at::Tensor>& found_inf) {
  fused_adamw_impl(params, grads, exp_avgs, exp_avg_sqs, max_exp_avg_sqs, state_steps, lr, at::Tensor(), beta1,
                   beta2, weight_decay, eps, amsgrad, maximize, grad_scale, found_inf);
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
  m.impl("_foreach_add_.Scalar", TORCH_FN(foreach_add_scalar_));
  m.impl("_foreach_add.Scalar", TORCH_FN(foreach_add_scalar));
  m.impl("_foreach_add_.List", TORCH_FN(foreach_add_list_));
  m.impl("_foreach_add.List", TORCH_FN(foreach_add_list));
  m.impl("_foreach_mul_.Scalar", TORCH_FN(foreach_mul_scalar_));
  m.impl("_foreach_mul.Scalar", TORCH_FN(foreach_mul_scalar));
  m.impl("_foreach_mul_.List", TORCH_FN(foreach_mul_list_));
  m.impl("_foreach_mul.List", TORCH_FN(foreach_mul_list));
  m.impl("_fused_adamw_", TORCH_FN(fused_adamw_));
  m.impl("_fused_adamw_.tensor_lr", TORCH_FN(fused_adamw_tensor_lr_));
  m.impl("_amp_foreach_non_finite_check_and_unscale_", TORCH_FN(amp_unscale_));
  m.impl("_amp_update_scale_", TORCH_FN(amp_update_scale_));
}
