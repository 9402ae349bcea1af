// PrivateUse1 registrations of max / min reductions with their indices:
// amax / amin, max.dim / min.dim, argmax / argmin and the full max() / min()
// -- what logsumexp, accuracy metrics and hand-written softmaxes call next to
// the loss path.  The reduced dims go last in a contiguous copy; long rows
// reduce in two launches of the same kernel (chunks, then the chunk winners).
#include <ATen/native/Resize.h>
#include <ATen/WrapDimUtils.h>
#include <torch/library.h>

#include <algorithm>
#include <tuple>

#include "common.h"

namespace supa {
namespace {

constexpr int64_t kExtChunk = 16384;     // elements per workgroup in the first of two launches
constexpr int64_t kExtTwoPassRow = 65536;  // rows longer than this (with few rows) take two launches

struct ExtResult {
  at::Tensor values, indices;
};

// Reduces `self` over `dims` (all dims when empty).
ExtResult argext(const at::Tensor& self, std::vector<int64_t> dims, bool keepdim, bool is_min, bool want_val,
                 bool want_idx, const char* name) {
  TORCH_CHECK(self.device().type() == kSupa, name, ": expected a supa tensor");
  TORCH_CHECK(!at::isComplexType(self.scalar_type()), name, ": complex inputs are not supported");
  const int64_t nd = self.dim();
  if (dims.empty()) {
    for (int64_t i = 0; i < nd; ++i) dims.push_back(i);
  } else {
    for (auto& d : dims) d = at::maybe_wrap_dim(d, std::max<int64_t>(nd, 1));
    std::sort(dims.begin(), dims.end());
    dims.erase(std::unique(dims.begin(), dims.end()), dims.end());
    if (nd == 0) dims.clear();
  }
  std::vector<bool> red(nd, false);
  for (int64_t d : dims) red[d] = true;
  int64_t inner = 1;
  for (int64_t d : dims) {
    TORCH_CHECK(self.size(d) > 0, name, "(): Expected reduction dim ", d, " to have non-zero size.");
    inner *= self.size(d);
  }
  TORCH_CHECK(self.numel() > 0 || !dims.empty() || nd > 0, name,
              "(): Expected reduction dim to be specified for input.numel() == 0.");
  if (nd == 0) TORCH_CHECK(self.numel() == 1, name, ": empty input");
  std::vector<int64_t> oshape, perm;
  for (int64_t i = 0; i < nd; ++i) {
    if (!red[i]) {
      oshape.push_back(self.size(i));
      perm.push_back(i);
    } else if (keepdim) {
      oshape.push_back(1);
    }
  }
  for (int64_t d : dims) perm.push_back(d);
  const auto dev = self.device().index();
  at::Tensor rows = nd == 0 ? self.reshape({1}) : self.permute(perm).contiguous();
  const int64_t outer = inner > 0 ? rows.numel() / inner : 0;
  ExtResult r;
  if (want_val) r.values = empty_supa(oshape, self.scalar_type(), dev);
  if (want_idx) r.indices = empty_supa(oshape, at::kLong, dev);
  if (outer == 0) return r;
  TORCH_CHECK(inner > 0, name, "(): Expected reduction dim to have non-zero size.");
  const int code = dtype_code(self.scalar_type());
  void* s = current_stream(dev);
  if (inner > kExtTwoPassRow && outer < 2048) {
    const int64_t nchunks = (inner + kExtChunk - 1) / kExtChunk;
    at::Tensor pv = empty_supa({outer, nchunks}, self.scalar_type(), dev);
    at::Tensor pi = empty_supa({outer, nchunks}, at::kLong, dev);
    check_status(supa_amd_argext_rows(rows.data_ptr(), code, nullptr, outer, inner, kExtChunk, is_min ? 1 : 0,
                                      pv.data_ptr(), pi.data_ptr<int64_t>(), s),
                 name);
    check_status(supa_amd_argext_rows(pv.data_ptr(), code, pi.data_ptr<int64_t>(), outer, nchunks, nchunks,
                                      is_min ? 1 : 0, want_val ? r.values.data_ptr() : nullptr,
                                      want_idx ? r.indices.data_ptr<int64_t>() : nullptr, s),
                 name);
  } else {
    check_status(supa_amd_argext_rows(rows.data_ptr(), code, nullptr, outer, inner, inner, is_min ? 1 : 0,
                                      want_val ? r.values.data_ptr() : nullptr,
                                      want_idx ? r.indices.data_ptr<int64_t>() : nullptr, s),
                 name);
  }
  return r;
}

void into(const at::Tensor& src, at::Tensor& out) {
  at::native::resize_output(out, src.sizes());
  out.copy_(src);
}

std::vector<int64_t> dim_list(at::IntArrayRef dim) { return std::vector<int64_t>(dim.begin(), dim.end()); }

at::Tensor amax(const at::Tensor& self, at::IntArrayRef dim, bool keepdim) {
  return argext(self, dim_list(dim), keepdim, false, true, false, "amax").values;
}
at::Tensor& amax_out(const at::Tensor& self, at::IntArrayRef dim, bool keepdim, at::Tensor& out) {
  into(argext(self, dim_list(dim), keepdim, false, true, false, "amax").values, out);
  return out;
}
at::Tensor amin(const at::Tensor& self, at::IntArrayRef dim, bool keepdim) {
  return argext(self, dim_list(dim), keepdim, true, true, false, "amin").values;
}
at::Tensor& amin_out(const at::Tensor& self, at::IntArrayRef dim, bool keepdim, at::Tensor& out) {
  into(argext(self, dim_list(dim), keepdim, true, true, false, "amin").values, out);
  return out;
}

std::tuple<at::Tensor, at::Tensor> max_dim(const at::Tensor& self, int64_t dim, bool keepdim) {
  ExtResult r = argext(self, {dim}, keepdim, false, true, true, "max");
  return {r.values, r.indices};
}
std::tuple<at::Tensor&, at::Tensor&> max_dim_out(const at::Tensor& self, int64_t dim, bool keepdim, at::Tensor& v,
                                                 at::Tensor& i) {
  ExtResult r = argext(self, {dim}, keepdim, false, true, true, "max");
  into(r.values, v);
  into(r.indices, i);
  return {v, i};
}
std::tuple<at::Tensor, at::Tensor> min_dim(const at::Tensor& self, int64_t dim, bool keepdim) {
  ExtResult r = argext(self, {dim}, keepdim, true, true, true, "min");
  return {r.values, r.indices};
}
std::tuple<at::Tensor&, at::Tensor&> min_dim_out(const at::Tensor& self, int64_t dim, bool keepdim, at::Tensor& v,
                                                 at::Tensor& i) {
  ExtResult r = argext(self, {dim}, keepdim, true, true, true, "min");
  into(r.values, v);
  into(r.indices, i);
  return {v, i};
}

// argmax / argmin: no dim -> the flattened tensor (keepdim gives all-ones dims)
at::Tensor arg_any(const at::Tensor& self, std::optional<int64_t> dim, bool keepdim, bool is_min, const char* name) {
  if (dim.has_value()) return argext(self, {*dim}, keepdim, is_min, false, true, name).indices;
  TORCH_CHECK(self.numel() > 0, name, "(): Expected reduction dim to be specified for input.numel() == 0.");
  at::Tensor idx = argext(self.reshape({-1}), {0}, false, is_min, false, true, name).indices;
  if (keepdim) {
    std::vector<int64_t> ones(self.dim(), 1);
    return idx.reshape(ones);
  }
  return idx;
}
at::Tensor argmax(const at::Tensor& self, std::optional<int64_t> dim, bool keepdim) {
  return arg_any(self, dim, keepdim, false, "argmax");
}
at::Tensor& argmax_out(const at::Tensor& self, std::optional<int64_t> dim, bool keepdim, at::Tensor& out) {
  into(arg_any(self, dim, keepdim, false, "argmax"), out);
  return out;
}
at::Tensor argmin(const at::Tensor& self, std::optional<int64_t> dim, bool keepdim) {
  return arg_any(self, dim, keepdim, true, "argmin");
}
at::Tensor& argmin_out(const at::Tensor& self, std::optional<int64_t> dim, bool keepdim, at::Tensor& out) {
  into(arg_any(self, dim, keepdim, true, "argmin"), out);
  return out;
}

// max() / min() over everything: a 0-dim tensor
at::Tensor full_ext(const at::Tensor& self, bool is_min, const char* name) {
  TORCH_CHECK(self.numel() > 0, name,
              "(): Expected reduction dim to be specified for input.numel() == 0. Specify the reduction dim "
              "with the 'dim' argument.");
  return argext(self.reshape({-1}), {0}, false, is_min, true, false, name).values;
}
at::Tensor max_all(const at::Tensor& self) { return full_ext(self, false, "max"); }
at::Tensor& max_all_out(const at::Tensor& self, at::Tensor& out) {
  into(full_ext(self, false, "max"), out);
  return out;
}
at::Tensor min_all(const at::Tensor& self) { return full_ext(self, true, "min"); }
at::Tensor& min_all_out(const at::Tensor& self, at::Tensor& out) {
  into(full_ext(self, true, "min"), out);
  return out;
}

}  // namespace
}  // namespace supa

TORCH_LIBRARY_IMPL(aten, PrivateUse1, m) {
  using namespace supa;
  m.impl("amax", TORCH_FN(amax));
  m.impl("amax.out", TORCH_FN(amax_out));
  m.impl("amin", TORCH_FN(amin));
  m.impl("amin.out", TORCH_FN(amin_out));
  m.impl("max.dim", TORCH_FN(max_dim));
  m.impl("max.dim_max", TORCH_FN(max_dim_out));
  m.impl("min.dim", TORCH_FN(min_dim));
  m.impl("min.dim_min", TORCH_FN(min_dim_out));
  m.impl("argmax", TORCH_FN(argmax));
  m.impl("argmax.out", TORCH_FN(argmax_out));
  m.impl("argmin", TORCH_FN(argmin));
  m.impl("argmin.out", TORCH_FN(argmin_out));
  m.impl("max", TORCH_FN(max_all));
  m.impl("max.unary_out", TORCH_FN(max_all_out));
  m.impl("min", TORCH_FN(min_all));
  m.impl("min.unary_out", TORCH_FN(min_all_out));
}
