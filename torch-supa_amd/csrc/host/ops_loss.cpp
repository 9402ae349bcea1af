// PrivateUse1 registrations of the loss path: sum/mean reductions,
// mse_loss / smooth_l1_loss / binary_cross_entropy_with_logits (forward with
// fused reductions, and the mse / smooth_l1 gradients), _log_softmax and
// _softmax with their backwards, nll_loss and nll_loss2d forward / backward.
//
// cross_entropy_loss is registered the way the reference registers it
// (SUPANativeFunctions::cross_entropy_loss, CrossEntropyLoss.cpp:140-151),
// with its routing: 2-d float32 logits with int64 class targets or a float32
// probability target of the logits' shape, no class weight and no label
// smoothing take the fused kernels (a custom autograd function, as the
// reference's CrossEntropyLossFastPathFunction); everything else, bfloat16 and
// float16 logits included, calls upstream's composite cross_entropy_loss_symint,
// i.e. the _log_softmax + nll_loss decomposition whose nested calls record
// autograd -- the path the reference takes for every non-fp32 input (:23-52).
// torch.supa.set_fused_cross_entropy_enabled(True / False) routes every
// floating dtype to the fused kernels, or none.
// binary_cross_entropy_with_logits is registered, as the reference registers
// it (supa_native_functions.yaml:59-61; BinaryCrossEntropyWithLogits.cpp:23-73);
// its backward is the autograd formula's op sequence on the kernels above.
#include <ATen/WrapDimUtils.h>
#include <ATen/ops/cross_entropy_loss_native.h>
#include <ATen/ops/log_sigmoid.h>
#include <torch/csrc/autograd/custom_function.h>
#include <ATen/native/Resize.h>
#include <ATen/native/TypeProperties.h>
#include <c10/core/ScalarType.h>
#include <torch/library.h>

#include "common.h"
#include "ew_apply.h"
#include "planner.h"

namespace supa {
namespace {

constexpr int64_t kNone = 0, kMean = 1, kSum = 2;  // at::Reduction

int reduction_code(int64_t r) {
  TORCH_CHECK(r == kNone || r == kMean || r == kSum, "invalid reduction enum: ", r);
  return r == kNone ? SUPA_AMD_REDUCTION_NONE : (r == kMean ? SUPA_AMD_REDUCTION_MEAN : SUPA_AMD_REDUCTION_SUM);
}

bool is_float_dtype(c10::ScalarType t) {
  return t == at::kFloat || t == at::kBFloat16 || t == at::kHalf || t == at::kDouble;
}

// Full reduction of f(inputs) over the broadcast iteration space into the
// one-element `out`, through a reduction entry point of the C ABI.
void reduce_apply(const at::Tensor& out, const std::vector<at::Tensor>& ins, c10::ScalarType common,
                  const std::function<int(const supa_amd_ew_desc*, void*, int64_t, void*)>& launch, const char* name) {
  std::vector<const at::Tensor*> ts{&out};
  for (const auto& t : ins) ts.push_back(&t);
  const c10::DeviceIndex dev = common_device(ts, name);
  std::vector<PlanOperand> pops(1 + ins.size());
  pops[0].is_output = true;
  pops[0].allocate = true;
  for (size_t i = 0; i < ins.size(); ++i) {
    pops[1 + i].sizes = ins[i].sizes().vec();
    pops[1 + i].strides = ins[i].strides().vec();
  }
  Plan plan;
  try {
    plan = make_plan(pops);
  } catch (const std::invalid_argument& e) {
    TORCH_CHECK(false, name, ": ", e.what());
  }
  TORCH_CHECK((int)plan.it_sizes.size() <= SUPA_AMD_MAX_DIMS, name, ": too many dimensions");
  supa_amd_ew_desc d{};
  d.ndim = (int32_t)plan.it_sizes.size();
  d.noperands = (int32_t)(1 + ins.size());
  d.common_dtype = dtype_code(common);
  for (int i = 0; i < d.ndim; ++i) d.sizes[i] = plan.it_sizes[i];
  d.op[0].data = out.data_ptr();
  d.op[0].dtype = dtype_code(out.scalar_type());
  for (size_t k = 0; k < ins.size(); ++k) {
    supa_amd_operand& o = d.op[1 + k];
    o.data = ins[k].data_ptr();
    o.dtype = dtype_code(ins[k].scalar_type());
    for (int i = 0; i < d.ndim; ++i) o.strides[i] = plan.it_strides[1 + k][i];
  }
  const auto prev = current_device();
  if (prev != dev) set_device(dev);
  // the two-stage reduction's partials: a per-call block of the stream-ordered
  // caching allocator (no content requirement)
  const int64_t ws_bytes = std::max(supa_amd_sum_workspace_bytes(0), supa_amd_loss_workspace_bytes(0));
  const at::Tensor ws = empty_supa({ws_bytes}, at::kByte, dev);
  const int rc = launch(&d, ws.data_ptr(), ws_bytes, current_stream(dev));
  if (prev != dev) set_device(prev);
  check_status(rc, name);
}

at::Tensor to_dtype(const at::Tensor& t, c10::ScalarType dt) { return t.scalar_type() == dt ? t : t.to(dt); }

// ------------------------------------------------------------ sum / mean
std::vector<int64_t> reduce_dims(const at::Tensor& self, at::OptionalIntArrayRef dim) {
  std::vector<int64_t> dims;
  const int64_t nd = self.dim();
  if (!dim.has_value() || dim->empty()) {
    for (int64_t i = 0; i < nd; ++i) dims.push_back(i);
  } else {
    for (int64_t d : *dim) dims.push_back(at::maybe_wrap_dim(d, std::max<int64_t>(nd, 1)));
    std::sort(dims.begin(), dims.end());
    dims.erase(std::unique(dims.begin(), dims.end()), dims.end());
  }
  if (nd == 0) dims.clear();
  return dims;
}

at::Tensor& sum_mean_into(const at::Tensor& self, at::OptionalIntArrayRef dim, bool keepdim,
                          std::optional<c10::ScalarType> dtype, bool mean, at::Tensor& out, const char* name) {
  c10::ScalarType acc_dt = dtype.value_or(self.scalar_type());
  const bool int_in = at::isIntegralType(self.scalar_type(), true);
  if (!dtype && int_in) acc_dt = at::kLong;
  // integer / bool sums accumulate in int64 (upstream's sum of integral
  // tensors); a floating dtype argument converts the input first
  const bool int_sum = !mean && int_in && acc_dt == at::kLong;
  TORCH_CHECK(int_sum || (is_float_dtype(acc_dt) && (int_in || is_float_dtype(self.scalar_type()))), name,
              ": supa implements floating-point reductions and integer sums (got ", self.scalar_type(), " -> ",
              acc_dt, ")");
  const std::vector<int64_t> dims = reduce_dims(self, dim);
  std::vector<int64_t> oshape;
  std::vector<bool> red(self.dim(), false);
  for (int64_t d : dims) red[d] = true;
  for (int64_t i = 0; i < self.dim(); ++i) {
    if (!red[i]) oshape.push_back(self.size(i));
    else if (keepdim) oshape.push_back(1);
  }
  if (out.defined()) {
    TORCH_CHECK(out.scalar_type() == acc_dt, name, ": expected out dtype ", acc_dt, " but got ", out.scalar_type());
    at::native::resize_output(out, oshape);
  } else {
    out = empty_supa(oshape, acc_dt, self.device().index());
  }
  int64_t nred = 1;
  for (int64_t d : dims) nred *= self.size(d);
  if (out.numel() == 0) return out;
  if (nred == 0) {
    out.fill_(mean ? std::numeric_limits<double>::quiet_NaN() : 0.0);
    return out;
  }
  const double scale = mean ? 1.0 / (double)nred : 1.0;
  // the input must hold the output dtype's family: promote once if asked
  at::Tensor x = self;
  if (int_in && !int_sum) x = self.to(acc_dt);
  else if (acc_dt == at::kDouble && self.scalar_type() != at::kDouble) x = self.to(at::kDouble);
  if ((int64_t)dims.size() == self.dim()) {
    at::Tensor res = out.is_contiguous() ? out : empty_supa({}, acc_dt, self.device().index());
    reduce_apply(res, {x}, x.scalar_type(),
                 [scale](const supa_amd_ew_desc* d, void* ws, int64_t wsb, void* s) {
                   return supa_amd_sum(d, scale, ws, wsb, s);
                 },
                 name);
    if (!res.is_same(out)) out.copy_(res.reshape(out.sizes()));
    return out;
  }
  // move the reduced dims last, make rows contiguous, reduce each row
  std::vector<int64_t> perm;
  for (int64_t i = 0; i < x.dim(); ++i)
    if (!red[i]) perm.push_back(i);
  for (int64_t d : dims) perm.push_back(d);
  at::Tensor rows = x.permute(perm).contiguous();
  const int64_t outer = rows.numel() / nred;
  at::Tensor res = out.is_contiguous() ? out : empty_supa(oshape, acc_dt, self.device().index());
  const int rc = supa_amd_sum_rows(rows.data_ptr(), dtype_code(rows.scalar_type()), res.data_ptr(),
                                   dtype_code(acc_dt), outer, nred, scale, current_stream(self.device().index()));
  check_status(rc, name);
  if (!res.is_same(out)) out.copy_(res);
  return out;
}

// all() / any() over every element: the count of nonzero elements (NaN
// counts, as upstream's truthiness) against numel / 0, by the device's compare
// and integer sum; a uint8 input gives a uint8 result, as upstream.
at::Tensor& all_any_into(const at::Tensor& self, bool any, at::Tensor& out, const char* name) {
  const c10::ScalarType odt = self.scalar_type() == at::kByte ? at::kByte : at::kBool;
  if (out.defined()) {
    TORCH_CHECK(out.scalar_type() == odt, name, ": expected out dtype ", odt, " but got ", out.scalar_type());
    at::native::resize_output(out, {});
  } else {
    out = empty_supa({}, odt, self.device().index());
  }
  at::Tensor cnt = at::ne(self, 0).sum();
  out.copy_(any ? at::gt(cnt, 0) : at::eq(cnt, self.numel()));
  return out;
}
at::Tensor all_all(const at::Tensor& self) {
  at::Tensor out;
  return all_any_into(self, false, out, "all");
}
at::Tensor& all_all_out(const at::Tensor& self, at::Tensor& out) { return all_any_into(self, false, out, "all.all_out"); }
at::Tensor any_all(const at::Tensor& self) {
  at::Tensor out;
  return all_any_into(self, true, out, "any");
}
at::Tensor& any_all_out(const at::Tensor& self, at::Tensor& out) { return all_any_into(self, true, out, "any.all_out"); }

at::Tensor sum_dim(const at::Tensor& self, at::OptionalIntArrayRef dim, bool keepdim,
                   std::optional<c10::ScalarType> dtype) {
  at::Tensor out;
  return sum_mean_into(self, dim, keepdim, dtype, false, out, "sum");
}
at::Tensor& sum_out(const at::Tensor& self, at::OptionalIntArrayRef dim, bool keepdim,
                    std::optional<c10::ScalarType> dtype, at::Tensor& out) {
  return sum_mean_into(self, dim, keepdim, dtype, false, out, "sum.IntList_out");
}
at::Tensor mean_dim(const at::Tensor& self, at::OptionalIntArrayRef dim, bool keepdim,
                    std::optional<c10::ScalarType> dtype) {
  at::Tensor out;
  return sum_mean_into(self, dim, keepdim, dtype, true, out, "mean");
}
at::Tensor& mean_out(const at::Tensor& self, at::OptionalIntArrayRef dim, bool keepdim,
                     std::optional<c10::ScalarType> dtype, at::Tensor& out) {
  return sum_mean_into(self, dim, keepdim, dtype, true, out, "mean.out");
}

// ------------------------------------------------------- pointwise losses
at::Tensor loss_forward(int loss, const at::Tensor& self, const at::Tensor& target, const at::Tensor& pos_weight,
                        const at::Tensor& weight, int64_t reduction, double beta, at::Tensor out, const char* name) {
  const int red = reduction_code(reduction);
  std::vector<at::Tensor> ins{self, target};
  if (pos_weight.defined()) ins.push_back(pos_weight);
  if (weight.defined()) ins.push_back(weight);
  at::native::ResultTypeState rts{};
  for (const auto& t : ins) rts = at::native::update_result_type_state(t, rts);
  const c10::ScalarType common = at::native::result_type(rts);
  TORCH_CHECK(is_float_dtype(common), name, ": expected a floating-point input, got ", common);
  const int has_pw = pos_weight.defined() ? 1 : 0, has_w = weight.defined() ? 1 : 0;
  if (red == SUPA_AMD_REDUCTION_NONE) {
    std::vector<EwIn> eins;
    for (const auto& t : ins) eins.push_back(EwIn::of(t));
    if (!out.defined() && loss == SUPA_AMD_LOSS_BCE_LOGITS) out = empty_supa(self.sizes(), common, self.device().index());
    return ew_apply(out, out.defined() ? out.scalar_type() : common, common, eins,
                    [loss, beta, has_pw, has_w](const supa_amd_ew_desc* d, void* s) {
                      return supa_amd_loss_forward(d, loss, SUPA_AMD_REDUCTION_NONE, beta, has_pw, has_w, nullptr,
                                                   nullptr, 0, s);
                    },
                    name);
  }
  const c10::ScalarType out_dt = out.defined() ? out.scalar_type() : common;
  if (out.defined()) at::native::resize_output(out, {});
  else out = empty_supa({}, out_dt, self.device().index());
  int64_t n = 1;
  for (int64_t s : at::infer_size(self.sizes(), target.sizes())) n *= s;
  if (n == 0) {
    out.fill_(red == SUPA_AMD_REDUCTION_MEAN ? std::numeric_limits<double>::quiet_NaN() : 0.0);
    return out;
  }
  for (auto& t : ins) t = to_dtype(t, common);
  at::Tensor res = out.scalar_type() == common ? out : empty_supa({}, common, self.device().index());
  reduce_apply(res, ins, common,
               [loss, red, beta, has_pw, has_w, &res](const supa_amd_ew_desc* d, void* ws, int64_t wsb, void* s) {
                 return supa_amd_loss_forward(d, loss, red, beta, has_pw, has_w, res.data_ptr(), ws, wsb, s);
               },
               name);
  if (!res.is_same(out)) out.copy_(res);
  return out;
}

at::Tensor mse_loss(const at::Tensor& self, const at::Tensor& target, int64_t reduction) {
  return loss_forward(SUPA_AMD_LOSS_MSE, self, target, {}, {}, reduction, 0.0, {}, "mse_loss");
}
at::Tensor& mse_loss_out(const at::Tensor& self, const at::Tensor& target, int64_t reduction, at::Tensor& out) {
  loss_forward(SUPA_AMD_LOSS_MSE, self, target, {}, {}, reduction, 0.0, out, "mse_loss.out");
  return out;
}
void check_beta(double beta) { TORCH_CHECK(beta >= 0, "smooth_l1_loss does not support negative values for beta."); }
at::Tensor smooth_l1_loss(const at::Tensor& self, const at::Tensor& target, int64_t reduction, double beta) {
  check_beta(beta);
  return loss_forward(SUPA_AMD_LOSS_SMOOTH_L1, self, target, {}, {}, reduction, beta, {}, "smooth_l1_loss");
}
at::Tensor& smooth_l1_loss_out(const at::Tensor& self, const at::Tensor& target, int64_t reduction, double beta,
                               at::Tensor& out) {
  check_beta(beta);
  loss_forward(SUPA_AMD_LOSS_SMOOTH_L1, self, target, {}, {}, reduction, beta, out, "smooth_l1_loss.out");
  return out;
}
at::Tensor bce_with_logits(const at::Tensor& self, const at::Tensor& target, const std::optional<at::Tensor>& weight,
                           const std::optional<at::Tensor>& pos_weight, int64_t reduction) {
  TORCH_CHECK(self.sizes() == target.sizes(), "Target size (", target.sizes(),
              ") must be the same as input size (", self.sizes(), ")");
  TORCH_CHECK(at::isFloatingType(self.scalar_type()),
              "binary_cross_entropy_with_logits is only implemented for floating dtypes");
  const at::Tensor pw = pos_weight.has_value() ? *pos_weight : at::Tensor();
  const at::Tensor w = weight.has_value() ? *weight : at::Tensor();
  return loss_forward(SUPA_AMD_LOSS_BCE_LOGITS, self, target, pw, w, reduction, 0.0, {},
                      "binary_cross_entropy_with_logits");
}

at::Tensor loss_backward(int loss, const at::Tensor& grad, const at::Tensor& self, const at::Tensor& target,
                         int64_t reduction, double beta, at::Tensor gi, const char* name,
                         const at::Tensor& weight = at::Tensor()) {
  reduction_code(reduction);
  at::native::ResultTypeState rts{};
  for (const at::Tensor* t : {&grad, &self, &target}) rts = at::native::update_result_type_state(*t, rts);
  if (weight.defined()) rts = at::native::update_result_type_state(weight, rts);
  const c10::ScalarType common = at::native::result_type(rts);
  TORCH_CHECK(is_float_dtype(common), name, ": expected a floating-point input, got ", common);
  int64_t n = 1;
  for (int64_t s : at::infer_size(self.sizes(), target.sizes())) n *= s;
  double norm;
  if (loss == SUPA_AMD_LOSS_MSE) norm = reduction == kMean ? 2.0 / (double)n : 2.0;
  else if (loss == SUPA_AMD_LOSS_BCE) norm = reduction == kMean ? (double)n : 1.0;  // the divisor
  else norm = reduction == kMean ? 1.0 / (double)n : 1.0;
  std::vector<EwIn> ins{EwIn::of(grad), EwIn::of(self), EwIn::of(target)};
  if (weight.defined()) ins.push_back(EwIn::of(weight));
  return ew_apply(gi, gi.defined() ? gi.scalar_type() : common, common, ins,
                  [loss, norm, beta](const supa_amd_ew_desc* d, void* s) {
                    return supa_amd_loss_backward(d, loss, norm, beta, s);
                  },
                  name);
}

at::Tensor mse_loss_backward(const at::Tensor& grad, const at::Tensor& self, const at::Tensor& target,
                             int64_t reduction) {
  return loss_backward(SUPA_AMD_LOSS_MSE, grad, self, target, reduction, 0.0, {}, "mse_loss_backward");
}
at::Tensor& mse_loss_backward_out(const at::Tensor& grad, const at::Tensor& self, const at::Tensor& target,
                                  int64_t reduction, at::Tensor& gi) {
  loss_backward(SUPA_AMD_LOSS_MSE, grad, self, target, reduction, 0.0, gi, "mse_loss_backward.grad_input");
  return gi;
}
at::Tensor smooth_l1_loss_backward(const at::Tensor& grad, const at::Tensor& self, const at::Tensor& target,
                                   int64_t reduction, double beta) {
  check_beta(beta);
  return loss_backward(SUPA_AMD_LOSS_SMOOTH_L1, grad, self, target, reduction, beta, {}, "smooth_l1_loss_backward");
}
at::Tensor& smooth_l1_loss_backward_out(const at::Tensor& grad, const at::Tensor& self, const at::Tensor& target,
                                        int64_t reduction, double beta, at::Tensor& gi) {
  check_beta(beta);
  loss_backward(SUPA_AMD_LOSS_SMOOTH_L1, grad, self, target, reduction, beta, gi,
                "smooth_l1_loss_backward.grad_input");
  return gi;
}

// huber_loss: smooth_l1's shape with delta (upstream huber_kernel_cuda,
// huber_backward_cuda_kernel)
void check_delta(double delta) {
  TORCH_CHECK(delta > 0, "huber_loss does not support non-positive values for delta.");
}
at::Tensor huber_loss(const at::Tensor& self, const at::Tensor& target, int64_t reduction, double delta) {
  check_delta(delta);
  return loss_forward(SUPA_AMD_LOSS_HUBER, self, target, {}, {}, reduction, delta, {}, "huber_loss");
}
at::Tensor& huber_loss_out(const at::Tensor& self, const at::Tensor& target, int64_t reduction, double delta,
                           at::Tensor& out) {
  check_delta(delta);
  loss_forward(SUPA_AMD_LOSS_HUBER, self, target, {}, {}, reduction, delta, out, "huber_loss.out");
  return out;
}
at::Tensor huber_loss_backward(const at::Tensor& grad, const at::Tensor& self, const at::Tensor& target,
                               int64_t reduction, double delta) {
  check_delta(delta);
  return loss_backward(SUPA_AMD_LOSS_HUBER, grad, self, target, reduction, delta, {}, "huber_loss_backward");
}
at::Tensor& huber_loss_backward_out(const at::Tensor& grad, const at::Tensor& self, const at::Tensor& target,
                                    int64_t reduction, double delta, at::Tensor& gi) {
  check_delta(delta);
  loss_backward(SUPA_AMD_LOSS_HUBER, grad, self, target, reduction, delta, gi, "huber_loss_backward.out");
  return gi;
}

// binary_cross_entropy on probabilities (upstream binary_cross_entropy_out /
// _backward): the input's values are not checked to lie in [0, 1] (that would
// need a device-to-host read); outside it the log is NaN.
void check_bce(const at::Tensor& self, const at::Tensor& target, const std::optional<at::Tensor>& weight) {
  TORCH_CHECK(self.sizes() == target.sizes(), "Using a target size (", target.sizes(),
              ") that is different to the input size (", self.sizes(), ") is deprecated. ",
              "Please ensure they have the same size.");
  TORCH_CHECK(at::isFloatingType(self.scalar_type()), "binary_cross_entropy is only implemented for floating dtypes");
  (void)weight;
}
at::Tensor bce_weight(const std::optional<at::Tensor>& weight) {
  return weight.has_value() && weight->defined() ? *weight : at::Tensor();
}
at::Tensor binary_cross_entropy(const at::Tensor& self, const at::Tensor& target,
                                const std::optional<at::Tensor>& weight, int64_t reduction) {
  check_bce(self, target, weight);
  at::Tensor out = empty_supa(self.sizes(), self.scalar_type(), self.device().index());
  if (reduction != kNone) out = at::Tensor();
  return loss_forward(SUPA_AMD_LOSS_BCE, self, target, {}, bce_weight(weight), reduction, 0.0, out,
                      "binary_cross_entropy");
}
at::Tensor& binary_cross_entropy_out(const at::Tensor& self, const at::Tensor& target,
                                     const std::optional<at::Tensor>& weight, int64_t reduction, at::Tensor& out) {
  check_bce(self, target, weight);
  loss_forward(SUPA_AMD_LOSS_BCE, self, target, {}, bce_weight(weight), reduction, 0.0, out,
               "binary_cross_entropy.out");
  return out;
}
at::Tensor binary_cross_entropy_backward(const at::Tensor& grad, const at::Tensor& self, const at::Tensor& target,
                                         const std::optional<at::Tensor>& weight, int64_t reduction) {
  check_bce(self, target, weight);
  at::Tensor gi = empty_supa(self.sizes(), self.scalar_type(), self.device().index());
  return loss_backward(SUPA_AMD_LOSS_BCE, grad, self, target, reduction, 0.0, gi, "binary_cross_entropy_backward",
                       bce_weight(weight));
}
at::Tensor& binary_cross_entropy_backward_out(const at::Tensor& grad, const at::Tensor& self,
                                              const at::Tensor& target, const std::optional<at::Tensor>& weight,
                                              int64_t reduction, at::Tensor& gi) {
  check_bce(self, target, weight);
  loss_backward(SUPA_AMD_LOSS_BCE, grad, self, target, reduction, 0.0, gi,
                "binary_cross_entropy_backward.grad_input", bce_weight(weight));
  return gi;
}

// ------------------------------------------------------------ log_softmax
// Runs `fn(rows, cols)` on contiguous row-major views with `dim` last; the
// result is returned in the original dim order, contiguous.
// log_softmax (LOG) and softmax share the layout handling: the reduced dim
// is moved last (a copy when it is not), rows run through the row kernels.
at::Tensor& softmax_into(bool log, const at::Tensor& self, int64_t dim, bool half_to_float, at::Tensor& out,
                         const char* name) {
  TORCH_CHECK(is_float_dtype(self.scalar_type()), name, ": expected a floating-point input, got ", self.scalar_type());
  if (half_to_float)
    TORCH_CHECK(self.scalar_type() == at::kHalf || self.scalar_type() == at::kBFloat16,
                "conversion is supported for Half and BFloat16 type only");
  const c10::ScalarType odt = half_to_float ? at::kFloat : self.scalar_type();
  const int64_t d = at::maybe_wrap_dim(dim, std::max<int64_t>(self.dim(), 1));
  if (out.defined()) {
    at::native::resize_output(out, self.sizes());
    TORCH_CHECK(out.scalar_type() == odt, name, ": expected out dtype ", odt);
  } else {
    out = empty_supa(self.sizes(), odt, self.device().index());
  }
  if (self.numel() == 0) return out;
  if (self.dim() == 0) {
    out.fill_(log ? 0 : 1);
    return out;
  }
  const bool last = d == self.dim() - 1;
  at::Tensor x = last ? self.contiguous() : self.movedim(d, -1).contiguous();
  const int64_t cols = x.size(-1);
  const int64_t rows = x.numel() / cols;
  at::Tensor res = (last && out.is_contiguous()) ? out : empty_supa(x.sizes(), odt, self.device().index());
  const auto fwd = log ? supa_amd_log_softmax_forward : supa_amd_softmax_forward;
  const int rc = fwd(x.data_ptr(), dtype_code(x.scalar_type()), res.data_ptr(), dtype_code(odt), rows, cols,
                     current_stream(self.device().index()));
  check_status(rc, name);
  if (!res.is_same(out)) out.copy_(last ? res : res.movedim(-1, d));
  return out;
}
at::Tensor log_softmax(const at::Tensor& self, int64_t dim, bool half_to_float) {
  at::Tensor out;
  return softmax_into(true, self, dim, half_to_float, out, "_log_softmax");
}
at::Tensor& log_softmax_out(const at::Tensor& self, int64_t dim, bool half_to_float, at::Tensor& out) {
  return softmax_into(true, self, dim, half_to_float, out, "_log_softmax.out");
}
at::Tensor softmax(const at::Tensor& self, int64_t dim, bool half_to_float) {
  at::Tensor out;
  return softmax_into(false, self, dim, half_to_float, out, "_softmax");
}
at::Tensor& softmax_out(const at::Tensor& self, int64_t dim, bool half_to_float, at::Tensor& out) {
  return softmax_into(false, self, dim, half_to_float, out, "_softmax.out");
}

at::Tensor& softmax_bwd_into(bool log, const at::Tensor& grad, const at::Tensor& output, int64_t dim,
                             c10::ScalarType input_dtype, at::Tensor& gi, const char* name) {
  TORCH_CHECK(grad.sizes() == output.sizes(), name, ": grad and output sizes differ");
  const int64_t d = at::maybe_wrap_dim(dim, std::max<int64_t>(grad.dim(), 1));
  if (gi.defined()) at::native::resize_output(gi, grad.sizes());
  else gi = empty_supa(grad.sizes(), input_dtype, grad.device().index());
  if (grad.numel() == 0) return gi;
  if (grad.dim() == 0) {
    gi.fill_(0);
    return gi;
  }
  const bool last = d == grad.dim() - 1;
  const c10::ScalarType gdt = at::promote_types(grad.scalar_type(), output.scalar_type());
  at::Tensor g = to_dtype(last ? grad.contiguous() : grad.movedim(d, -1).contiguous(), gdt);
  at::Tensor y = to_dtype(last ? output.contiguous() : output.movedim(d, -1).contiguous(), gdt);
  const int64_t cols = g.size(-1);
  const int64_t rows = g.numel() / cols;
  const c10::ScalarType kdt = (gi.scalar_type() == gdt) ? gdt : at::kFloat;
  at::Tensor res = (last && gi.is_contiguous() && gi.scalar_type() == kdt)
                       ? gi
                       : empty_supa(g.sizes(), kdt, grad.device().index());
  const auto bwd = log ? supa_amd_log_softmax_backward : supa_amd_softmax_backward;
  const int rc = bwd(g.data_ptr(), y.data_ptr(), dtype_code(gdt), res.data_ptr(), dtype_code(kdt), rows, cols,
                     current_stream(grad.device().index()));
  check_status(rc, name);
  if (!res.is_same(gi)) gi.copy_(last ? res : res.movedim(-1, d));
  return gi;
}
at::Tensor log_softmax_backward(const at::Tensor& grad, const at::Tensor& output, int64_t dim,
                                c10::ScalarType input_dtype) {
  at::Tensor gi;
  return softmax_bwd_into(true, grad, output, dim, input_dtype, gi, "_log_softmax_backward_data");
}
at::Tensor& log_softmax_backward_out(const at::Tensor& grad, const at::Tensor& output, int64_t dim,
                                     c10::ScalarType input_dtype, at::Tensor& gi) {
  return softmax_bwd_into(true, grad, output, dim, input_dtype, gi, "_log_softmax_backward_data.out");
}
at::Tensor softmax_backward(const at::Tensor& grad, const at::Tensor& output, int64_t dim,
                            c10::ScalarType input_dtype) {
  at::Tensor gi;
  return softmax_bwd_into(false, grad, output, dim, input_dtype, gi, "_softmax_backward_data");
}
at::Tensor& softmax_backward_out(const at::Tensor& grad, const at::Tensor& output, int64_t dim,
                                 c10::ScalarType input_dtype, at::Tensor& gi) {
  return softmax_bwd_into(false, grad, output, dim, input_dtype, gi, "_softmax_backward_data.out");
}

// --------------------------------------------------------------- nll_loss
void nll_checks(const at::Tensor& self, const at::Tensor& target, const at::Tensor& weight) {
  TORCH_CHECK(self.dim() > 0 && self.dim() <= 2, "input tensor should be 1D or 2D");
  TORCH_CHECK(target.dim() <= 1, "0D or 1D target tensor expected, multi-target not supported");
  const bool no_batch_dim = self.dim() == 1 && target.dim() == 0;
  TORCH_CHECK(no_batch_dim || (self.size(0) == target.size(0)), "size mismatch (got input: ", self.sizes(),
              ", target: ", target.sizes(), ")");
  TORCH_CHECK(target.scalar_type() == at::kLong, "nll_loss: expected target of scalar type Long but found ",
              target.scalar_type());
  const int64_t n_classes = self.size(-1);
  TORCH_CHECK(!weight.defined() || (weight.dim() == 1 && weight.numel() == n_classes),
              "weight tensor should be defined either for all ", n_classes,
              " classes or no classes but got weight tensor of shape: ", weight.sizes());
  TORCH_CHECK(is_float_dtype(self.scalar_type()), "nll_loss: expected a floating-point input");
}

std::tuple<at::Tensor&, at::Tensor&> nll_fwd_into(const at::Tensor& self, const at::Tensor& target,
                                                  const std::optional<at::Tensor>& weight_opt, int64_t reduction,
                                                  int64_t ignore_index, at::Tensor& out, at::Tensor& tw) {
  const at::Tensor weight = weight_opt.has_value() ? *weight_opt : at::Tensor();
  nll_checks(self, target, weight);
  const int red = reduction_code(reduction);
  const int64_t n = self.dim() == 1 ? 1 : self.size(0);
  const int64_t c = self.size(-1);
  const auto dev = self.device().index();
  std::vector<int64_t> oshape;
  if (red == SUPA_AMD_REDUCTION_NONE && self.dim() == 2) oshape = {n};
  if (out.defined()) at::native::resize_output(out, oshape);
  else out = empty_supa(oshape, self.scalar_type(), dev);
  if (tw.defined()) at::native::resize_output(tw, {});
  else tw = empty_supa({}, self.scalar_type(), dev);
  at::Tensor x = self.contiguous();
  at::Tensor t = target.contiguous();
  at::Tensor w = weight.defined() ? to_dtype(weight, self.scalar_type()).contiguous() : at::Tensor();
  if (red == SUPA_AMD_REDUCTION_NONE) tw.zero_();
  int32_t* const eflag = stream_error_flag(dev);
  const int rc = supa_amd_nll_loss_forward(x.data_ptr(), dtype_code(x.scalar_type()), t.data_ptr<int64_t>(),
                                           w.defined() ? w.data_ptr() : nullptr, n, c, red, ignore_index,
                                           out.data_ptr(), tw.data_ptr(), eflag, current_stream(dev));
  check_status(rc, "nll_loss_forward");
  return {out, tw};
}
std::tuple<at::Tensor, at::Tensor> nll_loss_forward(const at::Tensor& self, const at::Tensor& target,
                                                    const std::optional<at::Tensor>& weight, int64_t reduction,
                                                    int64_t ignore_index) {
  at::Tensor out, tw;
  nll_fwd_into(self, target, weight, reduction, ignore_index, out, tw);
  return {out, tw};
}
std::tuple<at::Tensor&, at::Tensor&> nll_loss_forward_out(const at::Tensor& self, const at::Tensor& target,
                                                          const std::optional<at::Tensor>& weight, int64_t reduction,
                                                          int64_t ignore_index, at::Tensor& out, at::Tensor& tw) {
  return nll_fwd_into(self, target, weight, reduction, ignore_index, out, tw);
}

at::Tensor& nll_bwd_into(const at::Tensor& grad, const at::Tensor& self, const at::Tensor& target,
                         const std::optional<at::Tensor>& weight_opt, int64_t reduction, int64_t ignore_index,
                         const at::Tensor& total_weight, at::Tensor& gi) {
  const at::Tensor weight = weight_opt.has_value() ? *weight_opt : at::Tensor();
  nll_checks(self, target, weight);
  const int red = reduction_code(reduction);
  const int64_t n = self.dim() == 1 ? 1 : self.size(0);
  const int64_t c = self.size(-1);
  const auto dev = self.device().index();
  if (gi.defined()) at::native::resize_output(gi, self.sizes());
  else gi = empty_supa(self.sizes(), self.scalar_type(), dev);
  TORCH_CHECK(total_weight.numel() == 1, "expected total_weight to be a single element tensor");
  at::Tensor res = gi.is_contiguous() ? gi : empty_supa(self.sizes(), self.scalar_type(), dev);
  at::Tensor g = to_dtype(grad, self.scalar_type()).contiguous();
  at::Tensor t = target.contiguous();
  at::Tensor w = weight.defined() ? to_dtype(weight, self.scalar_type()).contiguous() : at::Tensor();
  at::Tensor tw = to_dtype(total_weight, self.scalar_type());
  if (red == SUPA_AMD_REDUCTION_NONE && self.dim() == 2)
    TORCH_CHECK(g.numel() == n, "Expected a tensor of dimension 1 and tensor.size[0] == ", n);
  int32_t* const eflag = stream_error_flag(dev);
  const int rc = supa_amd_nll_loss_backward(g.data_ptr(), dtype_code(self.scalar_type()), t.data_ptr<int64_t>(),
                                            w.defined() ? w.data_ptr() : nullptr, tw.data_ptr(), n, c,
                                            red == SUPA_AMD_REDUCTION_NONE && self.dim() == 1 ? SUPA_AMD_REDUCTION_SUM
                                                                                               : red,
                                            ignore_index, res.data_ptr(), eflag, current_stream(dev));
  check_status(rc, "nll_loss_backward");
  if (!res.is_same(gi)) gi.copy_(res);
  return gi;
}
at::Tensor nll_loss_backward(const at::Tensor& grad, const at::Tensor& self, const at::Tensor& target,
                             const std::optional<at::Tensor>& weight, int64_t reduction, int64_t ignore_index,
                             const at::Tensor& total_weight) {
  at::Tensor gi;
  return nll_bwd_into(grad, self, target, weight, reduction, ignore_index, total_weight, gi);
}
at::Tensor& nll_loss_backward_out(const at::Tensor& grad, const at::Tensor& self, const at::Tensor& target,
                                  const std::optional<at::Tensor>& weight, int64_t reduction, int64_t ignore_index,
                                  const at::Tensor& total_weight, at::Tensor& gi) {
  return nll_bwd_into(grad, self, target, weight, reduction, ignore_index, total_weight, gi);
}

// ------------------------------------------------------------ nll_loss2d
// [N, C, H, W] log-probabilities with [N, H, W] targets (what
// cross_entropy uses for inputs of more than two dims) on the spatial nll
// kernels; the checks and messages are upstream's (LossNLL2d.cpp).
void nll2d_checks(const at::Tensor& self, const at::Tensor& target, const at::Tensor& weight) {
  TORCH_CHECK(target.dim() == 3, "only batches of spatial targets supported (3D tensors) but got targets of dimension: ",
              target.dim());
  TORCH_CHECK(self.dim() == 4, "only batches of spatial inputs supported (4D tensors), but got input of dimension: ",
              self.dim());
  TORCH_CHECK(!weight.defined() || weight.numel() == self.size(1),
              "weight tensor should be defined either for all or no classes");
  TORCH_CHECK(self.size(0) == target.size(0) && self.size(2) == target.size(1) && self.size(3) == target.size(2),
              "input and target batch or spatial sizes don't match: target ", target.sizes(), ", input ",
              self.sizes());
  TORCH_CHECK(target.scalar_type() == at::kLong, "nll_loss2d: expected target of scalar type Long but found ",
              target.scalar_type());
  TORCH_CHECK(is_float_dtype(self.scalar_type()), "nll_loss2d: expected a floating-point input");
}

std::tuple<at::Tensor&, at::Tensor&> nll2d_fwd_into(const at::Tensor& self, const at::Tensor& target,
                                                    const std::optional<at::Tensor>& weight_opt, int64_t reduction,
                                                    int64_t ignore_index, at::Tensor& out, at::Tensor& tw) {
  const at::Tensor weight = weight_opt.has_value() ? *weight_opt : at::Tensor();
  nll2d_checks(self, target, weight);
  const int red = reduction_code(reduction);
  const int64_t n = self.size(0), c = self.size(1), sp = self.size(2) * self.size(3);
  const auto dev = self.device().index();
  std::vector<int64_t> oshape;
  if (red == SUPA_AMD_REDUCTION_NONE) oshape = {n, self.size(2), self.size(3)};
  if (out.defined()) at::native::resize_output(out, oshape);
  else out = empty_supa(oshape, self.scalar_type(), dev);
  if (tw.defined()) at::native::resize_output(tw, {});
  else tw = empty_supa({}, self.scalar_type(), dev);
  at::Tensor x = self.contiguous();
  at::Tensor t = target.contiguous();
  at::Tensor w = weight.defined() ? to_dtype(weight, self.scalar_type()).contiguous() : at::Tensor();
  if (red == SUPA_AMD_REDUCTION_NONE) tw.zero_();
  at::Tensor res = out.is_contiguous() ? out : empty_supa(oshape, self.scalar_type(), dev);
  int32_t* const eflag = stream_error_flag(dev);
  const int64_t ws_bytes = supa_amd_nll_loss2d_workspace_bytes();
  const at::Tensor ws = empty_supa({ws_bytes}, at::kByte, dev);
  const int rc = supa_amd_nll_loss2d_forward(x.data_ptr(), dtype_code(x.scalar_type()), t.data_ptr<int64_t>(),
                                             w.defined() ? w.data_ptr() : nullptr, n, c, sp, red, ignore_index,
                                             res.data_ptr(), tw.data_ptr(), ws.data_ptr(), ws_bytes,
                                             eflag, current_stream(dev));
  check_status(rc, "nll_loss2d_forward");
  if (!res.is_same(out)) out.copy_(res);
  return {out, tw};
}
std::tuple<at::Tensor, at::Tensor> nll_loss2d_forward(const at::Tensor& self, const at::Tensor& target,
                                                      const std::optional<at::Tensor>& weight, int64_t reduction,
                                                      int64_t ignore_index) {
  at::Tensor out, tw;
  nll2d_fwd_into(self, target, weight, reduction, ignore_index, out, tw);
  return {out, tw};
}
std::tuple<at::Tensor&, at::Tensor&> nll_loss2d_forward_out(const at::Tensor& self, const at::Tensor& target,
                                                            const std::optional<at::Tensor>& weight,
                                                            int64_t reduction, int64_t ignore_index, at::Tensor& out,
                                                            at::Tensor& tw) {
  return nll2d_fwd_into(self, target, weight, reduction, ignore_index, out, tw);
}

at::Tensor& nll2d_bwd_into(const at::Tensor& grad, const at::Tensor& self, const at::Tensor& target,
                           const std::optional<at::Tensor>& weight_opt, int64_t reduction, int64_t ignore_index,
                           const at::Tensor& total_weight, at::Tensor& gi) {
  const at::Tensor weight = weight_opt.has_value() ? *weight_opt : at::Tensor();
  nll2d_checks(self, target, weight);
  const int red = reduction_code(reduction);
  const int64_t n = self.size(0), c = self.size(1), sp = self.size(2) * self.size(3);
  const auto dev = self.device().index();
  TORCH_CHECK(total_weight.numel() == 1, "expected total_weight to be a single element tensor, got: ",
              total_weight.sizes(), " (", total_weight.numel(), " elements)");
  if (red == SUPA_AMD_REDUCTION_NONE) {
    TORCH_CHECK(grad.dim() == 3 && grad.size(0) == n && grad.size(1) == self.size(2) && grad.size(2) == self.size(3),
                "nll_loss2d_backward: expected grad_output of size ", target.sizes(), ", got ", grad.sizes());
  } else {
    TORCH_CHECK(grad.numel() == 1, "nll_loss2d_backward: expected a single-element grad_output");
  }
  if (gi.defined()) at::native::resize_output(gi, self.sizes());
  else gi = empty_supa(self.sizes(), self.scalar_type(), dev);
  at::Tensor res = gi.is_contiguous() ? gi : empty_supa(self.sizes(), self.scalar_type(), dev);
  at::Tensor g = to_dtype(grad, self.scalar_type()).contiguous();
  at::Tensor t = target.contiguous();
  at::Tensor w = weight.defined() ? to_dtype(weight, self.scalar_type()).contiguous() : at::Tensor();
  at::Tensor tw = to_dtype(total_weight, self.scalar_type());
  int32_t* const eflag = stream_error_flag(dev);
  const int rc = supa_amd_nll_loss2d_backward(g.data_ptr(), dtype_code(self.scalar_type()), t.data_ptr<int64_t>(),
                                              w.defined() ? w.data_ptr() : nullptr, tw.data_ptr(), n, c, sp, red,
                                              ignore_index, res.data_ptr(), eflag, current_stream(dev));
  check_status(rc, "nll_loss2d_backward");
  if (!res.is_same(gi)) gi.copy_(res);
  return gi;
}
at::Tensor nll_loss2d_backward(const at::Tensor& grad, const at::Tensor& self, const at::Tensor& target,
                               const std::optional<at::Tensor>& weight, int64_t reduction, int64_t ignore_index,
                               const at::Tensor& total_weight) {
  at::Tensor gi;
  return nll2d_bwd_into(grad, self, target, weight, reduction, ignore_index, total_weight, gi);
}
at::Tensor& nll_loss2d_backward_out(const at::Tensor& grad, const at::Tensor& self, const at::Tensor& target,
                                    const std::optional<at::Tensor>& weight, int64_t reduction, int64_t ignore_index,
                                    const at::Tensor& total_weight, at::Tensor& gi) {
  return nll2d_bwd_into(grad, self, target, weight, reduction, ignore_index, total_weight, gi);
}

// ------------------------------------------ BCE-with-logits autograd
// binary_cross_entropy_with_logits' input gradient, the autograd formula
// (binary_cross_entropy_with_logits_backward of upstream's FunctionsManual;
// derivatives.yaml:2017-2019) op by op on this backend's kernels: used under
// create_graph (so the gradient is itself differentiable), for mixed dtypes,
// and when the fused kernel is switched off.
at::Tensor bce_input_grad_ops(const at::Tensor& g, const at::Tensor& self, const at::Tensor& target,
                              const at::Tensor& weight, const at::Tensor& pos_weight, int64_t reduction) {
  at::Tensor gi;
  if (pos_weight.defined()) {
    at::Tensor u = pos_weight.mul(target);
    gi = u.add(1).sub(target).mul(self.sigmoid()).sub(u);
  } else {
    gi = self.sigmoid().sub(target);
  }
  gi = gi.mul(g);
  if (weight.defined()) gi = gi.mul(weight);
  if (reduction == kMean) gi = gi.div(self.numel());
  return gi;
}

// binary_cross_entropy_with_logits_target_backward, op by op.
at::Tensor bce_target_grad_ops(const at::Tensor& g, const at::Tensor& self, const at::Tensor& target,
                               const at::Tensor& weight, const at::Tensor& pos_weight, int64_t reduction) {
  at::Tensor gt;
  if (pos_weight.defined()) gt = at::log_sigmoid(self.neg()).sub(at::log_sigmoid(self).mul(pos_weight)).mul(g);
  else gt = self.neg().mul(g);
  if (weight.defined()) gt = gt.mul(weight);
  if (reduction == kMean) gt = gt.div(target.numel());
  return gt;
}

// The same gradient in one kernel when every tensor shares one floating
// dtype (bit-identical: each intermediate is rounded to that dtype).
bool bce_fusable(const at::Tensor& g, const at::Tensor& self, const at::Tensor& target, const at::Tensor& weight,
                 const at::Tensor& pos_weight) {
  const auto dt = self.scalar_type();
  if (!fused_bce_backward_enabled() || !is_float_dtype(dt) || self.device().type() != c10::DeviceType::PrivateUse1)
    return false;
  for (const at::Tensor* t : {&g, &target, &weight, &pos_weight})
    if (t->defined() && (t->scalar_type() != dt || t->device() != self.device())) return false;
  return true;
}

at::Tensor bce_input_grad_fused(const at::Tensor& g, const at::Tensor& self, const at::Tensor& target,
                                const at::Tensor& weight, const at::Tensor& pos_weight, int64_t reduction) {
  std::vector<EwIn> ins{EwIn::of(g), EwIn::of(self), EwIn::of(target)};
  if (pos_weight.defined()) ins.push_back(EwIn::of(pos_weight));
  if (weight.defined()) ins.push_back(EwIn::of(weight));
  const int has_pw = pos_weight.defined() ? 1 : 0, has_w = weight.defined() ? 1 : 0;
  const int mean = reduction == kMean ? 1 : 0;
  const double numel = (double)self.numel();
  at::Tensor gi = ew_apply({}, self.scalar_type(), self.scalar_type(), ins,
                           [=](const supa_amd_ew_desc* d, void* st) {
                             return supa_amd_bce_logits_backward(d, has_pw, has_w, mean, numel, st);
                           },
                           "binary_cross_entropy_with_logits_backward");
  TORCH_CHECK(gi.sizes() == self.sizes(), "binary_cross_entropy_with_logits_backward: gradient shape ", gi.sizes(),
              " does not match the input ", self.sizes());
  return gi;
}

class BceWithLogitsFunction : public torch::autograd::Function<BceWithLogitsFunction> {
 public:
  // weight / pos_weight travel as optionals: an undefined at::Tensor is not a
  // valid autograd Function input
  static at::Tensor forward(torch::autograd::AutogradContext* ctx, const at::Tensor& self, const at::Tensor& target,
                            const std::optional<at::Tensor>& weight, const std::optional<at::Tensor>& pos_weight,
                            int64_t reduction) {
    at::Tensor out = bce_with_logits(self, target, weight, pos_weight, reduction);
    ctx->save_for_backward({self, target, weight.value_or(at::Tensor()), pos_weight.value_or(at::Tensor())});
    ctx->saved_data["reduction"] = reduction;
    return out;
  }

  static torch::autograd::variable_list backward(torch::autograd::AutogradContext* ctx,
                                                 torch::autograd::variable_list grads) {
    const auto saved = ctx->get_saved_variables();
    const at::Tensor& self = saved[0];
    const at::Tensor& target = saved[1];
    const at::Tensor& weight = saved[2];
    const at::Tensor& pos_weight = saved[3];
    const int64_t reduction = ctx->saved_data["reduction"].toInt();
    const at::Tensor& g = grads[0];
    at::Tensor gself, gtarget;
    if (ctx->needs_input_grad(0)) {
      if (!at::GradMode::is_enabled() && bce_fusable(g, self, target, weight, pos_weight))
        gself = bce_input_grad_fused(g, self, target, weight, pos_weight, reduction);
      else
        gself = bce_input_grad_ops(g, self, target, weight, pos_weight, reduction);
    }
    if (ctx->needs_input_grad(1)) gtarget = bce_target_grad_ops(g, self, target, weight, pos_weight, reduction);
    return {gself, gtarget, at::Tensor(), at::Tensor(), at::Tensor()};
  }
};

// The autograd-key kernel: weight and pos_weight have no derivative upstream
// either.
at::Tensor bce_with_logits_autograd(const at::Tensor& self, const at::Tensor& target,
                                    const std::optional<at::Tensor>& weight,
                                    const std::optional<at::Tensor>& pos_weight, int64_t reduction) {
  const bool w = weight.has_value() && weight->defined();
  const bool pw = pos_weight.has_value() && pos_weight->defined();
  TORCH_CHECK(!(w && weight->requires_grad()), "the derivative for 'weight' is not implemented.");
  TORCH_CHECK(!(pw && pos_weight->requires_grad()), "the derivative for 'pos_weight' is not implemented.");
  return BceWithLogitsFunction::apply(self, target, w ? weight : std::nullopt, pw ? pos_weight : std::nullopt,
                                      reduction);
}

// ------------------------------------------------------ fused cross-entropy
// The routing of CrossEntropyLoss.cpp:23-33 (supported_fast_path): 2-d logits,
// no class weight, no label smoothing, a valid reduction, and an int64 class
// target [n] or a probability target of the logits' shape.  The reference
// takes it for float32; the routing mode widens it to every floating dtype
// or turns it off.  A probability target must have the logits' dtype and
// need no gradient (the fused backward writes the logits' gradient only);
// its ignore_index must be negative, as the reference checks (other cases go
// to the composite, which raises upstream's error).
bool fused_ce_dtype_on(at::ScalarType dt) {
  const int mode = fused_cross_entropy_mode();
  if (mode == 0) return false;
  if (mode < 0) return dt == at::kFloat;
  return dt == at::kFloat || dt == at::kBFloat16 || dt == at::kHalf;
}

bool fused_ce_base(const at::Tensor& self, const at::Tensor& target, const std::optional<at::Tensor>& weight,
                   int64_t reduction, double label_smoothing) {
  return fused_ce_dtype_on(self.scalar_type()) && self.dim() == 2 && !(weight.has_value() && weight->defined()) &&
         label_smoothing == 0.0 && target.device() == self.device() &&
         (reduction == at::Reduction::None || reduction == at::Reduction::Mean || reduction == at::Reduction::Sum);
}

bool fused_ce_supported(const at::Tensor& self, const at::Tensor& target, const std::optional<at::Tensor>& weight,
                        int64_t reduction, double label_smoothing) {
  return fused_ce_base(self, target, weight, reduction, label_smoothing) && target.dim() == 1 &&
         target.scalar_type() == at::kLong && target.size(0) == self.size(0);
}

bool fused_ce_prob_supported(const at::Tensor& self, const at::Tensor& target,
                             const std::optional<at::Tensor>& weight, int64_t reduction, int64_t ignore_index,
                             double label_smoothing) {
  return fused_ce_base(self, target, weight, reduction, label_smoothing) && target.sizes() == self.sizes() &&
         target.scalar_type() == self.scalar_type() && !target.requires_grad() && ignore_index < 0;
}

class FusedCrossEntropy : public torch::autograd::Function<FusedCrossEntropy> {
 public:
  static at::Tensor forward(torch::autograd::AutogradContext* ctx, const at::Tensor& self, const at::Tensor& target,
                            int64_t reduction, int64_t ignore_index) {
    const int red = reduction_code(reduction);
    const int64_t n = self.size(0), c = self.size(1);
    TORCH_CHECK(c > 0, "cross_entropy: expected at least one class");
    const auto dev = self.device().index();
    at::Tensor x = self.contiguous();
    at::Tensor t = target.contiguous();
    at::Tensor out = empty_supa(red == SUPA_AMD_REDUCTION_NONE ? std::vector<int64_t>{n} : std::vector<int64_t>{},
                                self.scalar_type(), dev);
    at::Tensor lse = empty_supa({n}, at::kFloat, dev);
    at::Tensor count = empty_supa({}, at::kFloat, dev);
    at::Tensor ws = empty_supa({std::max<int64_t>(n, 1)}, at::kFloat, dev);
    int32_t* const eflag = stream_error_flag(dev);
    const int rc = supa_amd_cross_entropy_forward(x.data_ptr(), dtype_code(x.scalar_type()), t.data_ptr<int64_t>(), n,
                                                  c, ignore_index, red, out.data_ptr(), lse.data_ptr<float>(),
                                                  count.data_ptr<float>(), ws.data_ptr(), ws.numel() * 4,
                                                  eflag, current_stream(dev));
    check_status(rc, "cross_entropy (fused forward)");
    ctx->save_for_backward({x, t, lse, count});
    ctx->saved_data["reduction"] = reduction;
    ctx->saved_data["ignore_index"] = ignore_index;
    return out;
  }

  static torch::autograd::variable_list backward(torch::autograd::AutogradContext* ctx,
                                                 torch::autograd::variable_list grads) {
    const auto saved = ctx->get_saved_variables();
    const at::Tensor& x = saved[0];
    const at::Tensor& t = saved[1];
    const at::Tensor& lse = saved[2];
    const at::Tensor& count = saved[3];
    const int red = reduction_code(ctx->saved_data["reduction"].toInt());
    const int64_t ignore_index = ctx->saved_data["ignore_index"].toInt();
    const int64_t n = x.size(0), c = x.size(1);
    const auto dev = x.device().index();
    if (at::GradMode::is_enabled()) {
      // create_graph: the same gradient from differentiable ops,
      // (softmax(x) - onehot(t)) g_i over the kept rows
      const at::Tensor kept = ((t != ignore_index) * (t >= 0) * (t < c)).to(x.scalar_type());
      const at::Tensor oh = at::one_hot(t.clamp(0, c - 1), c).to(x.scalar_type());
      at::Tensor gr = red == SUPA_AMD_REDUCTION_NONE ? grads[0] : grads[0].expand({n});
      gr = gr * kept;
      if (red == SUPA_AMD_REDUCTION_MEAN) gr = gr / count.to(x.scalar_type());
      return {(at::softmax(x, 1, x.scalar_type()) - oh) * gr.unsqueeze(1), at::Tensor(), at::Tensor(),
              at::Tensor()};
    }
    at::Tensor g = to_dtype(grads[0], x.scalar_type()).contiguous();
    at::Tensor gx = empty_supa(x.sizes(), x.scalar_type(), dev);
    int32_t* const eflag = stream_error_flag(dev);
    const int rc = supa_amd_cross_entropy_backward(g.data_ptr(), x.data_ptr(), dtype_code(x.scalar_type()),
                                                   t.data_ptr<int64_t>(), lse.data_ptr<float>(),
                                                   count.data_ptr<float>(), n, c, ignore_index, red, gx.data_ptr(),
                                                   eflag, current_stream(dev));
    check_status(rc, "cross_entropy (fused backward)");
    return {gx, at::Tensor(), at::Tensor(), at::Tensor()};
  }
};

// Probability targets: loss_i = sum_j t_ij (lse_i - x_ij), as the
// reference's cross_entropy_prob_kernel (CrossEntropyLossKernel.cu:532-576);
// the backward is its prob_target branch (CrossEntropyLoss.cpp:94-131),
// -t g through _log_softmax_backward_data, in one pass:
// g_i (softmax(x_i) sum_j t_ij - t_i).
class FusedCrossEntropyProb : public torch::autograd::Function<FusedCrossEntropyProb> {
 public:
  static at::Tensor forward(torch::autograd::AutogradContext* ctx, const at::Tensor& self, const at::Tensor& target,
                            int64_t reduction) {
    const int red = reduction_code(reduction);
    const int64_t n = self.size(0), c = self.size(1);
    TORCH_CHECK(c > 0, "cross_entropy: expected at least one class");
    const auto dev = self.device().index();
    at::Tensor x = self.contiguous();
    at::Tensor t = target.contiguous();
    at::Tensor out = empty_supa(red == SUPA_AMD_REDUCTION_NONE ? std::vector<int64_t>{n} : std::vector<int64_t>{},
                                self.scalar_type(), dev);
    at::Tensor lse = empty_supa({n}, at::kFloat, dev);
    at::Tensor tsum = empty_supa({n}, at::kFloat, dev);
    at::Tensor ws = empty_supa({std::max<int64_t>(n, 1)}, at::kFloat, dev);
    const int rc = supa_amd_cross_entropy_prob_forward(x.data_ptr(), t.data_ptr(), dtype_code(x.scalar_type()), n, c,
                                                       red, out.data_ptr(), lse.data_ptr<float>(),
                                                       tsum.data_ptr<float>(), ws.data_ptr(), ws.numel() * 4,
                                                       current_stream(dev));
    check_status(rc, "cross_entropy (fused forward, probability target)");
    ctx->save_for_backward({x, t, lse, tsum});
    ctx->saved_data["reduction"] = reduction;
    return out;
  }

  static torch::autograd::variable_list backward(torch::autograd::AutogradContext* ctx,
                                                 torch::autograd::variable_list grads) {
    const auto saved = ctx->get_saved_variables();
    const at::Tensor& x = saved[0];
    const at::Tensor& t = saved[1];
    const at::Tensor& lse = saved[2];
    const at::Tensor& tsum = saved[3];
    const int red = reduction_code(ctx->saved_data["reduction"].toInt());
    const int64_t n = x.size(0), c = x.size(1);
    const auto dev = x.device().index();
    if (at::GradMode::is_enabled()) {
      // create_graph: (softmax(x) sum_j t_j - t) g_i from differentiable ops
      at::Tensor gr = red == SUPA_AMD_REDUCTION_NONE ? grads[0] : grads[0].expand({n});
      if (red == SUPA_AMD_REDUCTION_MEAN) gr = gr / (double)n;
      const at::Tensor p = at::softmax(x, 1, x.scalar_type());
      return {(p * t.sum(1, true) - t) * gr.unsqueeze(1), at::Tensor(), at::Tensor()};
    }
    at::Tensor g = to_dtype(grads[0], x.scalar_type()).contiguous();
    at::Tensor gx = empty_supa(x.sizes(), x.scalar_type(), dev);
    const int rc = supa_amd_cross_entropy_prob_backward(g.data_ptr(), x.data_ptr(), t.data_ptr(),
                                                        dtype_code(x.scalar_type()), lse.data_ptr<float>(),
                                                        tsum.data_ptr<float>(), n, c, red, gx.data_ptr(),
                                                        current_stream(dev));
    check_status(rc, "cross_entropy (fused backward, probability target)");
    return {gx, at::Tensor(), at::Tensor()};
  }
};

at::Tensor cross_entropy_loss(const at::Tensor& self, const at::Tensor& target,
                              const std::optional<at::Tensor>& weight, int64_t reduction, c10::SymInt ignore_index,
                              double label_smoothing) {
  if (fused_ce_supported(self, target, weight, reduction, label_smoothing))
    return FusedCrossEntropy::apply(self, target, reduction, ignore_index.expect_int());
  if (fused_ce_prob_supported(self, target, weight, reduction, ignore_index.expect_int(), label_smoothing))
    return FusedCrossEntropyProb::apply(self, target, reduction);
  return at::native::cross_entropy_loss_symint(self, target, weight, reduction, std::move(ignore_index),
                                               label_smoothing);
}

}  // namespace
}  // namespace supa

TORCH_LIBRARY_IMPL(aten, PrivateUse1, m) {
  using namespace supa;
  m.impl("sum.dim_IntList", TORCH_FN(sum_dim));
  m.impl("all", TORCH_FN(all_all));
  m.impl("all.all_out", TORCH_FN(all_all_out));
  m.impl("any", TORCH_FN(any_all));
  m.impl("any.all_out", TORCH_FN(any_all_out));
  m.impl("sum.IntList_out", TORCH_FN(sum_out));
  m.impl("mean.dim", TORCH_FN(mean_dim));
  m.impl("mean.out", TORCH_FN(mean_out));
  m.impl("mse_loss", TORCH_FN(mse_loss));
  m.impl("mse_loss.out", TORCH_FN(mse_loss_out));
  m.impl("mse_loss_backward", TORCH_FN(mse_loss_backward));
  m.impl("mse_loss_backward.grad_input", TORCH_FN(mse_loss_backward_out));
  m.impl("smooth_l1_loss", TORCH_FN(smooth_l1_loss));
  m.impl("smooth_l1_loss.out", TORCH_FN(smooth_l1_loss_out));
  m.impl("smooth_l1_loss_backward", TORCH_FN(smooth_l1_loss_backward));
  m.impl("smooth_l1_loss_backward.grad_input", TORCH_FN(smooth_l1_loss_backward_out));
  m.impl("huber_loss", TORCH_FN(huber_loss));
  m.impl("huber_loss.out", TORCH_FN(huber_loss_out));
  m.impl("huber_loss_backward", TORCH_FN(huber_loss_backward));
  m.impl("huber_loss_backward.out", TORCH_FN(huber_loss_backward_out));
  m.impl("binary_cross_entropy", TORCH_FN(binary_cross_entropy));
  m.impl("binary_cross_entropy.out", TORCH_FN(binary_cross_entropy_out));
  m.impl("binary_cross_entropy_backward", TORCH_FN(binary_cross_entropy_backward));
  m.impl("binary_cross_entropy_backward.grad_input", TORCH_FN(binary_cross_entropy_backward_out));
  m.impl("binary_cross_entropy_with_logits", TORCH_FN(bce_with_logits));
  m.impl("_log_softmax", TORCH_FN(log_softmax));
  m.impl("_log_softmax.out", TORCH_FN(log_softmax_out));
  m.impl("_log_softmax_backward_data", TORCH_FN(log_softmax_backward));
  m.impl("_log_softmax_backward_data.out", TORCH_FN(log_softmax_backward_out));
  m.impl("_softmax", TORCH_FN(softmax));
  m.impl("_softmax.out", TORCH_FN(softmax_out));
  m.impl("_softmax_backward_data", TORCH_FN(softmax_backward));
  m.impl("_softmax_backward_data.out", TORCH_FN(softmax_backward_out));
  m.impl("nll_loss_forward", TORCH_FN(nll_loss_forward));
  m.impl("nll_loss_forward.output", TORCH_FN(nll_loss_forward_out));
  m.impl("nll_loss_backward", TORCH_FN(nll_loss_backward));
  m.impl("nll_loss_backward.grad_input", TORCH_FN(nll_loss_backward_out));
  m.impl("nll_loss2d_forward", TORCH_FN(nll_loss2d_forward));
  m.impl("nll_loss2d_forward.output", TORCH_FN(nll_loss2d_forward_out));
  m.impl("nll_loss2d_backward", TORCH_FN(nll_loss2d_backward));
  m.impl("nll_loss2d_backward.grad_input", TORCH_FN(nll_loss2d_backward_out));
  m.impl("cross_entropy_loss", TORCH_FN(cross_entropy_loss));
}

// cross_entropy_loss has no autograd formula of its own (it is composite), so
// the autograd key needs the same kernel: the fused path attaches its own
// backward, and the composite path records autograd through its nested
// _log_softmax / nll_loss calls, as under the reference's autograd
// fallthrough (VariableFallbackKernel.cpp:31-33).
TORCH_LIBRARY_IMPL(aten, AutogradPrivateUse1, m) {
  m.impl("cross_entropy_loss", TORCH_FN(supa::cross_entropy_loss));
  // one-pass input gradient (bit-identical to the formula's op sequence)
  m.impl("binary_cross_entropy_with_logits", TORCH_FN(supa::bce_with_logits_autograd));
}
