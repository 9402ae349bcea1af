// PrivateUse1 registrations of var / std / var_mean / std_mean with a
// correction (what var(unbiased=...), std(), and LayerNorm or BatchNorm
// written out by hand resolve to).  The reduced dims go last in a contiguous
// copy and one row kernel returns the variance or standard deviation, and the
// mean beside it, for every row.  Complex and integer inputs go to the CPU
// fallback, which counts them (upstream raises for integers).
#include <ATen/WrapDimUtilsMulti.h>
#include <ATen/native/CPUFallback.h>
#include <ATen/native/Resize.h>
#include <ATen/ops/std_mean_ops.h>
#include <ATen/ops/std_ops.h>
#include <ATen/ops/var_mean_ops.h>
#include <ATen/ops/var_ops.h>
#include <torch/library.h>

#include <bitset>
#include <limits>
#include <tuple>

#include "common.h"

namespace supa {
namespace {

bool moments_dtype_ok(c10::ScalarType t) {
  return t == at::kFloat || t == at::kBFloat16 || t == at::kHalf || t == at::kDouble;
}

struct MomentsResult {
  at::Tensor var, mean;
};

MomentsResult moments(const at::Tensor& self, at::OptionalIntArrayRef dim, const std::optional<c10::Scalar>& correction,
                      bool keepdim, bool take_sqrt, bool want_mean, const char* name) {
  TORCH_CHECK(self.device().type() == kSupa, name, ": expected a supa tensor");
  const double corr = correction.has_value() ? correction->toDouble() : 1.0;
  const int64_t nd = self.dim();
  std::bitset<at::dim_bitset_size> red;
  if (!dim.has_value() || dim->empty()) {
    for (int64_t i = 0; i < nd; ++i) red.set(i);
  } else {
    red = at::dim_list_to_bitset(*dim, nd);  // wraps, and rejects repeated dims
  }
  std::vector<int64_t> oshape, perm;
  int64_t inner = 1, outer = 1;
  for (int64_t i = 0; i < nd; ++i) {
    if (!red[i]) {
      oshape.push_back(self.size(i));
      perm.push_back(i);
      outer *= self.size(i);
    } else if (keepdim) {
      oshape.push_back(1);
    }
  }
  for (int64_t i = 0; i < nd; ++i) {
    if (red[i]) {
      perm.push_back(i);
      inner *= self.size(i);
    }
  }
  if (static_cast<double>(inner) - corr <= 0.0) {
    TORCH_WARN(name, "(): degrees of freedom is <= 0. Correction should be strictly less than the reduction factor "
                     "(input numel divided by output numel).");
  }
  const auto opts = self.options();
  MomentsResult r;
  r.var = at::empty(oshape, opts);
  if (want_mean) r.mean = at::empty(oshape, opts);
  if (outer == 0) return r;
  if (inner == 0) {  // an empty reduction: NaN mean and variance
    r.var.fill_(std::numeric_limits<double>::quiet_NaN());
    if (want_mean) r.mean.fill_(std::numeric_limits<double>::quiet_NaN());
    return r;
  }
  const at::Tensor rows = nd == 0 ? self.reshape({1}) : self.permute(perm).contiguous();
  const int32_t dt = dtype_code(self.scalar_type());
  const int64_t ws_bytes = supa_amd_moments_rows_workspace_bytes(outer, inner, dt);
  TORCH_CHECK(ws_bytes >= 0, name, ": ", supa_amd_status_string((int)ws_bytes));
  at::Tensor ws;
  if (ws_bytes > 0) ws = at::empty({ws_bytes}, opts.dtype(at::kByte));
  check_status(supa_amd_moments_rows(rows.data_ptr(), dt, outer, inner, corr, take_sqrt ? 1 : 0, r.var.data_ptr(),
                                     want_mean ? r.mean.data_ptr() : nullptr, ws_bytes > 0 ? ws.data_ptr() : nullptr,
                                     ws_bytes, current_stream(self.device().index())),
               name);
  return r;
}

at::Tensor var_corr(const at::Tensor& self, at::OptionalIntArrayRef dim, const std::optional<c10::Scalar>& correction,
                    bool keepdim) {
  if (!moments_dtype_ok(self.scalar_type()))
    return at::native::call_fallback_fn<&supa_cpu_fallback, at::_ops::var_correction>::call(self, dim, correction,
                                                                                         keepdim);
  return moments(self, dim, correction, keepdim, false, false, "var").var;
}

at::Tensor std_corr(const at::Tensor& self, at::OptionalIntArrayRef dim, const std::optional<c10::Scalar>& correction,
                    bool keepdim) {
  if (!moments_dtype_ok(self.scalar_type()))
    return at::native::call_fallback_fn<&supa_cpu_fallback, at::_ops::std_correction>::call(self, dim, correction,
                                                                                         keepdim);
  return moments(self, dim, correction, keepdim, true, false, "std").var;
}

void into(const at::Tensor& src, at::Tensor& out, const char* name) {
  TORCH_CHECK(out.scalar_type() == src.scalar_type(), name, ": expected out dtype ", src.scalar_type(), ", got ",
              out.scalar_type());
  at::native::resize_output(out, src.sizes());
  out.copy_(src);
}

at::Tensor& var_corr_out(const at::Tensor& self, at::OptionalIntArrayRef dim,
                         const std::optional<c10::Scalar>& correction, bool keepdim, at::Tensor& out) {
  into(var_corr(self, dim, correction, keepdim), out, "var");
  return out;
}

at::Tensor& std_corr_out(const at::Tensor& self, at::OptionalIntArrayRef dim,
                         const std::optional<c10::Scalar>& correction, bool keepdim, at::Tensor& out) {
  into(std_corr(self, dim, correction, keepdim), out, "std");
  return out;
}

std::tuple<at::Tensor, at::Tensor> var_mean_corr(const at::Tensor& self, at::OptionalIntArrayRef dim,
                                                 const std::optional<c10::Scalar>& correction, bool keepdim) {
  if (!moments_dtype_ok(self.scalar_type()))
    return at::native::call_fallback_fn<&supa_cpu_fallback, at::_ops::var_mean_correction>::call(
        self, dim, correction, keepdim);
  MomentsResult r = moments(self, dim, correction, keepdim, false, true, "var_mean");
  return {r.var, r.mean};
}

std::tuple<at::Tensor, at::Tensor> std_mean_corr(const at::Tensor& self, at::OptionalIntArrayRef dim,
                                                 const std::optional<c10::Scalar>& correction, bool keepdim) {
  if (!moments_dtype_ok(self.scalar_type()))
    return at::native::call_fallback_fn<&supa_cpu_fallback, at::_ops::std_mean_correction>::call(
        self, dim, correction, keepdim);
  MomentsResult r = moments(self, dim, correction, keepdim, true, true, "std_mean");
  return {r.var, r.mean};
}

}  // namespace
}  // namespace supa

TORCH_LIBRARY_IMPL(aten, PrivateUse1, m) {
  using namespace supa;
  m.impl("var.correction", TORCH_FN(var_corr));
  m.impl("var.correction_out", TORCH_FN(var_corr_out));
  m.impl("std.correction", TORCH_FN(std_corr));
  m.impl("std.correction_out", TORCH_FN(std_corr_out));
  m.impl("var_mean.correction", TORCH_FN(var_mean_corr));
  m.impl("std_mean.correction", TORCH_FN(std_mean_corr));
}
