// PrivateUse1 registrations of the random ops beside the activation path:
// uniform_, normal_ (what randn / randn_like run), bernoulli_.float and
// native_dropout / native_dropout_backward
// (what F.dropout runs on this device), on the Philox kernels with the
// device generator's (seed, offset).  Other dtypes and the other random ops
// take the counted CPU fallback.
#include <ATen/native/CPUFallback.h>
#include <ATen/ops/bernoulli_ops.h>
#include <ATen/ops/normal_ops.h>
#include <ATen/ops/uniform_ops.h>
#include <torch/library.h>

#include "common.h"
#include "ew_apply.h"
#include "generator.h"

namespace supa {
namespace {

bool rng_dtype(c10::ScalarType t) { return t == at::kFloat || t == at::kBFloat16 || t == at::kHalf; }

// Runs `fill` on a contiguous buffer shaped like `self`, then copies back
// when `self` is not contiguous itself.
template <typename F>
void fill_dense(at::Tensor& self, F&& fill) {
  if (self.is_contiguous()) return fill(self);
  at::Tensor tmp = at::empty(self.sizes(), self.options());
  fill(tmp);
  self.copy_(tmp);
}

at::Tensor& uniform_(at::Tensor& self, double from, double to, std::optional<at::Generator> gen) {
  if (!rng_dtype(self.scalar_type()))
    return at::native::call_fallback_fn<&supa_cpu_fallback, at::_ops::uniform_>::call(self, from, to, gen);
  TORCH_CHECK(from <= to, "uniform_ expects to return a [from, to) range, but found from=", from, " > to=", to);
  if (self.numel() == 0) return self;
  const auto dev = self.device().index();
  const auto [seed, offset] = philox_inputs(gen, dev);
  fill_dense(self, [&](at::Tensor& t) {
    check_status(supa_amd_uniform(t.data_ptr(), dtype_code(t.scalar_type()), t.numel(), from, to, seed, offset,
                                  current_stream(dev)),
                 "uniform_");
  });
  return self;
}

at::Tensor& normal_(at::Tensor& self, double mean, double stdv, std::optional<at::Generator> gen) {
  if (!rng_dtype(self.scalar_type()))
    return at::native::call_fallback_fn<&supa_cpu_fallback, at::_ops::normal_>::call(self, mean, stdv, gen);
  TORCH_CHECK(stdv >= 0.0, "normal expects std >= 0.0, but found std ", stdv);
  if (self.numel() == 0) return self;
  const auto dev = self.device().index();
  const auto [seed, offset] = philox_inputs(gen, dev);
  fill_dense(self, [&](at::Tensor& t) {
    check_status(supa_amd_normal(t.data_ptr(), dtype_code(t.scalar_type()), t.numel(), mean, stdv, seed, offset,
                                 current_stream(dev)),
                 "normal_");
  });
  return self;
}

at::Tensor& bernoulli_float_(at::Tensor& self, double p, std::optional<at::Generator> gen) {
  if (!rng_dtype(self.scalar_type()))
    return at::native::call_fallback_fn<&supa_cpu_fallback, at::_ops::bernoulli__float>::call(self, p, gen);
  TORCH_CHECK(0 <= p && p <= 1, "bernoulli_ expects p to be in [0, 1], but got p=", p);
  if (self.numel() == 0) return self;
  const auto dev = self.device().index();
  const auto [seed, offset] = philox_inputs(gen, dev);
  fill_dense(self, [&](at::Tensor& t) {
    check_status(supa_amd_bernoulli(t.data_ptr(), dtype_code(t.scalar_type()), t.numel(), p, seed, offset,
                                    current_stream(dev)),
                 "bernoulli_");
  });
  return self;
}

// bernoulli_(p_tensor) (upstream bernoulli_tensor_cuda_kernel: 1 where a
// uniform draw in [0, 1) is below p): the draws come from the device's
// Philox stream through uniform_, the comparison and the cast are device
// kernels too.
at::Tensor& bernoulli_tensor_(at::Tensor& self, const at::Tensor& p, std::optional<at::Generator> gen) {
  TORCH_CHECK(rng_dtype(self.scalar_type()) || self.scalar_type() == at::kBool ||
                  at::isIntegralType(self.scalar_type(), false),
              "bernoulli_: unsupported dtype ", self.scalar_type());
  if (self.numel() == 0) return self;
  at::Tensor u = at::empty(self.sizes(), self.options().dtype(at::kFloat));
  u.uniform_(0.0, 1.0, gen);
  self.copy_(at::lt(u, p.to(self.device())));
  return self;
}

// upstream native_dropout_cuda: train == false -> (clone, ones); p == 1 ->
// zeros; otherwise keep with probability 1 - p and scale by 1 / (1 - p).
std::tuple<at::Tensor, at::Tensor> native_dropout(const at::Tensor& input, double p, std::optional<bool> train) {
  TORCH_CHECK(p >= 0 && p <= 1, "dropout probability has to be between 0 and 1, but got ", p);
  const auto bool_opts = input.options().dtype(at::kBool);
  if (train.has_value() && !train.value()) return {input.clone(), at::ones_like(input, bool_opts)};
  if (p == 1) return {at::zeros_like(input), at::zeros_like(input, bool_opts)};
  TORCH_CHECK(rng_dtype(input.scalar_type()), "native_dropout: supa supports float32, bfloat16 and float16, got ",
              input.scalar_type());
  at::Tensor x = input.contiguous();
  at::Tensor out = at::empty(x.sizes(), x.options());
  at::Tensor mask = at::empty(x.sizes(), bool_opts);
  if (x.numel() == 0) return {out, mask};
  const auto dev = x.device().index();
  const auto [seed, offset] = philox_inputs(std::nullopt, dev);
  check_status(supa_amd_dropout(x.data_ptr(), dtype_code(x.scalar_type()), out.data_ptr(),
                                reinterpret_cast<uint8_t*>(mask.data_ptr()), x.numel(), 1.0 - p, seed, offset,
                                current_stream(dev)),
               "native_dropout");
  return {out, mask};
}

at::Tensor native_dropout_backward(const at::Tensor& grad, const at::Tensor& mask, double scale) {
  TORCH_CHECK(mask.scalar_type() == at::kBool, "Mask should be Bool Scalar Type", mask.scalar_type());
  const EwLaunch fn = [scale](const supa_amd_ew_desc* d, void* s) { return supa_amd_mask_scale(d, scale, s); };
  return ew_apply(at::Tensor(), grad.scalar_type(), grad.scalar_type(), {EwIn::of(mask), EwIn::of(grad)}, fn,
                  "native_dropout_backward");
}

}  // namespace
}  // namespace supa

TORCH_LIBRARY_IMPL(aten, PrivateUse1, m) {
  using namespace supa;
  m.impl("uniform_", TORCH_FN(uniform_));
  m.impl("normal_", TORCH_FN(normal_));
  m.impl("bernoulli_.float", TORCH_FN(bernoulli_float_));
  m.impl("bernoulli_.Tensor", TORCH_FN(bernoulli_tensor_));
  m.impl("native_dropout", TORCH_FN(native_dropout));
  m.impl("native_dropout_backward", TORCH_FN(native_dropout_backward));
}
