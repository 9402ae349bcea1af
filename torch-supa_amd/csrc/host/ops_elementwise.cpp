// PrivateUse1 registrations of the tensor plumbing (factories, views, copies,
// fill) and of the elementwise operators: add/sub/rsub, mul, div (all rounding
// modes), the activation family and its gradients.
//
// Registration surface: TORCH_LIBRARY_IMPL(aten, PrivateUse1, m), the same
// one the reference's generated RegisterSUPANative*.cpp use
// (script/codegen_native/gen.py:106-195, :553-585), with the functional,
// in-place and out= overload of each op registered by hand.  The kernels these
// ops end in replace add_stub (UfuncCUDA_add.cu:341-345), mul_stub
// (BinaryMulKernel.cu:43), div_*_stub (BinaryDiv{True,Trunc,Floor}Kernel.cu)
// and the upstream activation kernels the reference takes from its operator
// library.
#include <ATen/EmptyTensor.h>
#include <ATen/ExpandUtils.h>
#include <ATen/MemoryOverlap.h>
#include <ATen/native/Resize.h>
#include <ATen/native/ResizeCommon.h>
#include <ATen/native/TensorFactories.h>
#include <ATen/ops/as_strided_native.h>
#include <ATen/ops/view_native.h>
#include <ATen/ops/_reshape_alias_native.h>
#include <c10/core/ScalarType.h>
#include <ATen/native/TypeProperties.h>
#include <torch/library.h>

#include <stdexcept>

#include "common.h"
#include "ew_apply.h"

namespace supa {

// ------------------------------------------------------------ ew_apply
EwIn EwIn::of(const at::Tensor& x) {
  EwIn e;
  if (x.device().is_cpu() && x.dim() == 0) {
    e.scalar = true;
    e.value = x.item();
  } else {
    e.t = x;
  }
  return e;
}

c10::DeviceIndex common_device(const std::vector<const at::Tensor*>& ts, const char* name) {
  c10::DeviceIndex dev = -1;
  for (const at::Tensor* t : ts) {
    if (!t || !t->defined()) continue;
    if (t->device().type() == kSupa) {
      const auto d = t->device().index();
      TORCH_CHECK(dev < 0 || dev == d, name, ": expected all tensors on the same supa device, got supa:", int(dev),
                  " and supa:", int(d));
      dev = d;
    } else {
      TORCH_CHECK(t->device().is_cpu() && t->dim() == 0, name,
                  ": expected all tensors to be on the same device, but found a ", t->device(), " tensor");
    }
  }
  return dev < 0 ? current_device() : dev;
}

at::Tensor ew_apply(at::Tensor out, c10::ScalarType out_dtype, c10::ScalarType common_dtype,
                    const std::vector<EwIn>& ins, const EwLaunch& launch, const char* name) {
  TORCH_CHECK(dtype_supported(common_dtype), name, ": dtype ", common_dtype, " is not supported on supa");
  std::vector<const at::Tensor*> ts;
  if (out.defined()) ts.push_back(&out);
  for (const EwIn& e : ins)
    if (!e.scalar) ts.push_back(&e.t);
  const c10::DeviceIndex dev = common_device(ts, name);
  for (const EwIn& e : ins)
    if (!e.scalar) TORCH_CHECK(dtype_supported(e.t.scalar_type()), name, ": dtype ", e.t.scalar_type(), " is not supported on supa");

  std::vector<PlanOperand> pops(1 + ins.size());
  for (size_t i = 0; i < ins.size(); ++i) {
    PlanOperand& p = pops[1 + i];
    if (ins[i].scalar) {
      p.scalar = true;
    } else {
      p.sizes = ins[i].t.sizes().vec();
      p.strides = ins[i].t.strides().vec();
    }
  }
  pops[0].is_output = true;
  std::vector<int64_t> shape;
  try {
    if (out.defined()) {
      pops[0].sizes = out.sizes().vec();
      pops[0].strides = out.strides().vec();
    }
    shape = broadcast_shape(pops);
  } catch (const std::invalid_argument& e) {
    TORCH_CHECK(false, name, ": ", e.what());
  }
  if (out.defined()) {
    TORCH_CHECK(dtype_supported(out.scalar_type()), name, ": output dtype ", out.scalar_type(), " is not supported on supa");
    if (out.sizes().vec() != shape) {
      at::native::resize_output(out, shape);
    }
    pops[0].sizes = out.sizes().vec();
    pops[0].strides = out.strides().vec();
  } else {
    pops[0].allocate = true;
  }
  Plan plan;
  try {
    plan = make_plan(pops);
  } catch (const std::invalid_argument& e) {
    TORCH_CHECK(false, name, ": ", e.what());
  }
  if (!out.defined()) {
    out = empty_strided_supa(plan.shape, plan.out_strides[0], out_dtype, dev);
  } else {
    at::assert_no_internal_overlap(out);
    for (const EwIn& e : ins)
      if (!e.scalar) at::assert_no_partial_overlap(out, e.t);
  }
  if (plan.numel == 0) return out;
  TORCH_CHECK((int)plan.it_sizes.size() <= SUPA_AMD_MAX_DIMS, name, ": more than ", SUPA_AMD_MAX_DIMS,
              " non-coalescable dimensions");
  TORCH_CHECK((int)(1 + ins.size()) <= SUPA_AMD_MAX_OPERANDS, name, ": too many operands");

  supa_amd_ew_desc d{};
  d.ndim = (int32_t)plan.it_sizes.size();
  d.noperands = (int32_t)(1 + ins.size());
  d.common_dtype = dtype_code(common_dtype);
  for (int i = 0; i < d.ndim; ++i) d.sizes[i] = plan.it_sizes[i];
  for (int k = 0; k < d.noperands; ++k) {
    supa_amd_operand& o = d.op[k];
    if (k > 0 && ins[k - 1].scalar) {
      const c10::Scalar& v = ins[k - 1].value;
      TORCH_CHECK(!v.isComplex(), name, ": complex scalars are not supported on supa");
      o.is_scalar = 1;
      o.dtype = dtype_code(common_dtype);
      if (v.isBoolean()) {
        o.scalar = v.toBool() ? 1.0 : 0.0;
        o.iscalar = v.toBool() ? 1 : 0;
      } else if (v.isIntegral(false)) {
        o.iscalar = v.toLong();
        o.scalar = static_cast<double>(o.iscalar);
      } else {
        o.scalar = v.toDouble();
        o.iscalar = static_cast<int64_t>(o.scalar);
      }
      continue;
    }
    const at::Tensor& t = k == 0 ? out : ins[k - 1].t;
    o.data = t.data_ptr();
    o.dtype = dtype_code(t.scalar_type());
    for (int i = 0; i < d.ndim; ++i) o.strides[i] = plan.it_strides[k][i];
  }
  const auto prev = current_device();
  if (prev != dev) set_device(dev);
  const int rc = launch(&d, current_stream(dev));
  if (prev != dev) set_device(prev);
  check_status(rc, name);
  return out;
}

namespace {

// -------------------------------------------------------------- helpers
c10::ScalarType default_float() { return c10::typeMetaToScalarType(c10::get_default_dtype()); }

void check_cast(c10::ScalarType common, const at::Tensor& out, const char* name) {
  TORCH_CHECK(c10::canCast(common, out.scalar_type()), name, ": result type ", common,
              " can't be cast to the desired output type ", out.scalar_type());
}

// ----------------------------------------------------- factories / views
// Under torch.use_deterministic_algorithms(True) with
// torch.utils.deterministic.fill_uninitialized_memory (its default), new
// tensors are filled with NaN (floating types) or the type's maximum
// (integers), as the reference's empty / empty_strided
// (torch_supa/csrc/aten/common/TensorFactories.cpp:18-50) and upstream's.
bool deterministic_fill() {
  return C10_UNLIKELY(at::globalContext().deterministicAlgorithms() &&
                      at::globalContext().deterministicFillUninitializedMemory());
}

at::Tensor empty_memory_format(c10::IntArrayRef size, std::optional<c10::ScalarType> dtype,
                               std::optional<c10::Layout> layout, std::optional<c10::Device> device,
                               std::optional<bool> pin_memory, std::optional<c10::MemoryFormat> fmt) {
  TORCH_CHECK(!layout || *layout == c10::Layout::Strided, "supa: only strided tensors are supported");
  TORCH_CHECK(!pin_memory || !*pin_memory, "supa: pin_memory applies to CPU tensors only");
  const auto dt = dtype.value_or(default_float());
  const c10::DeviceIndex dev = device && device->has_index() ? device->index() : current_device();
  at::Tensor t = empty_supa(size, dt, dev, fmt.value_or(c10::MemoryFormat::Contiguous));
  if (deterministic_fill()) at::native::fill_empty_deterministic_(t);
  return t;
}

at::Tensor empty_strided(c10::IntArrayRef size, c10::IntArrayRef stride, std::optional<c10::ScalarType> dtype,
                         std::optional<c10::Layout> layout, std::optional<c10::Device> device,
                         std::optional<bool> pin_memory) {
  TORCH_CHECK(!layout || *layout == c10::Layout::Strided, "supa: only strided tensors are supported");
  const auto dt = dtype.value_or(default_float());
  const c10::DeviceIndex dev = device && device->has_index() ? device->index() : current_device();
  at::Tensor t = empty_strided_supa(size, stride, dt, dev);
  if (deterministic_fill()) at::native::fill_empty_deterministic_(t);
  return t;
}

const at::Tensor& resize_(const at::Tensor& self, c10::IntArrayRef size, std::optional<c10::MemoryFormat> fmt) {
  c10::TensorImpl* impl = self.unsafeGetTensorImpl();
  if (self.sizes() == size && !fmt) return self;
  const int64_t old_numel = self.numel();
  (void)old_numel;
  impl->set_sizes_contiguous(size);
  const size_t needed =
      at::detail::computeStorageNbytesContiguous(size, self.dtype().itemsize(), impl->storage_offset());
  const c10::Storage& storage = impl->unsafe_storage();
  const int64_t old_nbytes = (int64_t)storage.nbytes();
  if (needed > storage.nbytes()) {
    TORCH_CHECK(storage.resizable(), "supa: trying to resize storage that is not resizable");
    at::detail::getPrivateUse1Hooks().resizePrivateUse1Bytes(storage, needed);
  }
  if (fmt) impl->empty_tensor_restride(*fmt);
  // the bytes a grown storage adds, as upstream's resize_
  if (deterministic_fill()) at::native::fill_resize_deterministic_(self, old_nbytes);
  return self;
}

// Copies between the supa device and the host, and within the device.
at::Tensor copy_from(const at::Tensor& self, const at::Tensor& dst, bool /*non_blocking*/) {
  TORCH_CHECK(self.defined() && dst.defined(), "supa copy: undefined tensor");
  if (dst.numel() == 0) return dst;
  const bool src_dev = self.device().type() == kSupa;
  const bool dst_dev = dst.device().type() == kSupa;
  if (src_dev && dst_dev) {
    TORCH_CHECK(self.device() == dst.device(), "supa copy across devices is not supported");
    if (self.scalar_type() == dst.scalar_type() && self.sizes() == dst.sizes() && self.strides() == dst.strides() &&
        self.is_non_overlapping_and_dense()) {
      if (self.data_ptr() != dst.data_ptr())
        SUPA_HIP_CHECK(hipMemcpyAsync(dst.data_ptr(), self.data_ptr(), dst.nbytes(), hipMemcpyDeviceToDevice,
                                      current_stream(dst.device().index())));
      return dst;
    }
    TORCH_CHECK(dtype_supported(self.scalar_type()) && dtype_supported(dst.scalar_type()),
                "supa copy: unsupported dtype");
    at::Tensor src = self;
    if (at::has_internal_overlap(dst) == at::MemOverlap::Yes) TORCH_CHECK(false, "supa copy: destination overlaps itself");
    if (at::get_overlap_status(self, dst) == at::MemOverlapStatus::Partial) src = self.clone();
    EwIn in;
    in.t = src.expand(dst.sizes());
    ew_apply(dst, dst.scalar_type(), src.scalar_type(), {in},
             [](const supa_amd_ew_desc* d, void* s) { return supa_amd_copy(d, s); }, "copy_");
    return dst;
  }
  if (dst_dev) {  // host -> device
    TORCH_CHECK(self.device().is_cpu(), "supa copy: unsupported source device ", self.device());
    if (dst.is_contiguous()) {
      at::Tensor h = self.to(dst.scalar_type()).expand(dst.sizes()).contiguous();
      memcpy_h2d(dst.data_ptr(), h.data_ptr(), dst.nbytes(), dst.device().index());
    } else {
      at::Tensor tmp = empty_supa(dst.sizes(), dst.scalar_type(), dst.device().index());
      copy_from(self, tmp, false);
      copy_from(tmp, dst, false);
    }
    return dst;
  }
  // device -> host
  TORCH_CHECK(dst.device().is_cpu(), "supa copy: unsupported destination device ", dst.device());
  const auto dev = self.device().index();
  at::Tensor src = self;
  if (!src.is_contiguous()) {
    at::Tensor tmp = empty_supa(src.sizes(), src.scalar_type(), dev);
    copy_from(src, tmp, false);
    src = tmp;
  }
  if (dst.is_contiguous() && dst.scalar_type() == src.scalar_type() && dst.sizes() == src.sizes()) {
    memcpy_d2h(dst.data_ptr(), src.data_ptr(), dst.nbytes(), dev);
  } else {
    at::Tensor h = at::empty(src.sizes(), src.options().device(at::kCPU));
    memcpy_d2h(h.data_ptr(), src.data_ptr(), h.nbytes(), dev);
    dst.copy_(h);
  }
  check_device_errors(dev);  // the kernels that produced src are done
  return dst;
}

// equal (upstream cuda_equal): same shape, then every element equal (so a
// NaN makes it false) by the device's compare and all(); an alias of itself
// with the same view is equal without a launch.
bool equal(const at::Tensor& self, const at::Tensor& other) {
  TORCH_CHECK(self.device() == other.device(), "Cannot compare two tensors on different devices. Got: ",
              self.device(), " and ", other.device());
  if (self.sizes() != other.sizes()) return false;
  if (self.numel() == 0) return true;
  if (self.is_alias_of(other) && self.storage_offset() == other.storage_offset() && self.dtype() == other.dtype() &&
      self.strides() == other.strides() && self.is_neg() == other.is_neg() && self.is_conj() == other.is_conj())
    return true;
  return at::eq(self, other).all().item<bool>();
}

// scatter_(dim, index, value) with upstream's shape checks (ScatterGatherChecks.h)
// and the assign form of scatter_fill_kernel; an index outside the
// destination's dim sets the device error flag, reported at the next sync.
at::Tensor& scatter_value_(at::Tensor& self, int64_t dim, const at::Tensor& index, const c10::Scalar& value) {
  TORCH_CHECK(index.scalar_type() == at::kLong, "scatter_(): Expected dtype int64 for index");
  TORCH_CHECK(self.device() == index.device(), "scatter_: expected self and index on the same device, got ",
              self.device(), " and ", index.device());
  const int64_t nd = std::max<int64_t>(self.dim(), 1);
  TORCH_CHECK(std::max<int64_t>(index.dim(), 1) == nd,
              "Index tensor must have the same number of dimensions as self tensor");
  const int64_t wd = at::maybe_wrap_dim(dim, nd);
  if (index.numel() == 0) return self;
  at::Tensor out = self.dim() == 0 ? self.view({1}) : self;
  at::Tensor idx = index.dim() == 0 ? index.view({1}) : index;
  for (int64_t d = 0; d < nd; ++d) {
    if (d == wd) continue;
    TORCH_CHECK(idx.size(d) <= out.size(d), "Expected index ", index.sizes(), " to be smaller than self ",
                self.sizes(), " apart from dimension ", wd);
  }
  TORCH_CHECK(nd <= SUPA_AMD_MAX_DIMS, "scatter_: supa supports up to ", SUPA_AMD_MAX_DIMS, " dimensions");
  TORCH_CHECK(dtype_supported(self.scalar_type()), "scatter_: unsupported dtype ", self.scalar_type());
  at::assert_no_internal_overlap(self);
  // the value in the destination's type, as upstream's value.to<scalar_t>()
  // (a checked conversion: an integer destination refuses a value it cannot
  // hold; a bool destination takes value != 0)
  int64_t ivalue = 0;
  switch (self.scalar_type()) {
    case at::kBool: ivalue = value.to<bool>() ? 1 : 0; break;
    case at::kByte: ivalue = value.to<uint8_t>(); break;
    case at::kChar: ivalue = value.to<int8_t>(); break;
    case at::kShort: ivalue = value.to<int16_t>(); break;
    case at::kInt: ivalue = value.to<int32_t>(); break;
    case at::kLong: ivalue = value.to<int64_t>(); break;
    default: break;  // floating destinations take the double
  }
  const auto dev = self.device().index();
  const int rc = supa_amd_scatter_fill(out.data_ptr(), dtype_code(out.scalar_type()), out.strides().data(),
                                       out.size(wd), idx.data_ptr<int64_t>(), idx.sizes().data(),
                                       idx.strides().data(), (int32_t)nd, (int32_t)wd, value.toDouble(), ivalue,
                                       stream_error_flag(dev), current_stream(dev));
  check_status(rc, "scatter_");
  return self;
}
at::Tensor scatter_value(const at::Tensor& self, int64_t dim, const at::Tensor& index, const c10::Scalar& value) {
  at::Tensor out = self.clone(at::MemoryFormat::Preserve);
  return scatter_value_(out, dim, index, value);
}
at::Tensor& scatter_value_out(const at::Tensor& self, int64_t dim, const at::Tensor& index, const c10::Scalar& value,
                              at::Tensor& out) {
  if (!out.is_same(self)) {
    at::native::resize_output(out, self.sizes());
    out.copy_(self);
  }
  return scatter_value_(out, dim, index, value);
}

// eye.out / eye.m_out (upstream eye_out_cuda): zeros, then ones on the
// diagonal through a strided view of it.
at::Tensor& eye_m_out(int64_t n, int64_t m, at::Tensor& out) {
  TORCH_CHECK(n >= 0, "n must be greater or equal to 0, got ", n);
  TORCH_CHECK(m >= 0, "m must be greater or equal to 0, got ", m);
  at::native::resize_output(out, {n, m});
  out.zero_();
  const int64_t sz = std::min<int64_t>(n, m);
  if (sz > 0) out.as_strided({sz}, {out.stride(0) + out.stride(1)}).fill_(1);
  return out;
}
at::Tensor& eye_out(int64_t n, at::Tensor& out) { return eye_m_out(n, n, out); }

at::Tensor copy_from_and_resize(const at::Tensor& self, const at::Tensor& dst) {
  if (dst.sizes() != self.sizes()) {
    if (dst.device().type() == kSupa) resize_(dst, self.sizes(), std::nullopt);
    else dst.resize_(self.sizes());
  }
  return copy_from(self, dst, false);
}

// upstream _local_scalar_dense reads the element at the data pointer with no
// size check (item() checks numel before it calls this)
c10::Scalar local_scalar_dense(const at::Tensor& self) {
  TORCH_CHECK(self.numel() > 0, "_local_scalar_dense: the tensor has no elements");
  at::Tensor h = at::empty({}, self.options().device(at::kCPU));
  memcpy_d2h(h.data_ptr(), self.data_ptr(), self.dtype().itemsize(), self.device().index());
  check_device_errors(self.device().index());
  return h.item();
}

at::Tensor& fill_scalar(at::Tensor& self, const c10::Scalar& value) {
  ew_apply(self, self.scalar_type(), self.scalar_type(), {EwIn::num(value)},
           [](const supa_amd_ew_desc* d, void* s) { return supa_amd_fill(d, s); }, "fill_");
  return self;
}

at::Tensor& fill_tensor(at::Tensor& self, const at::Tensor& value) {
  TORCH_CHECK(value.dim() == 0, "fill_ only supports 0-dimension value tensor but got tensor with ", value.dim(),
              " dimensions.");
  if (value.device().type() == kSupa) {
    EwIn in;
    in.t = value.expand(self.sizes());
    ew_apply(self, self.scalar_type(), value.scalar_type(), {in},
             [](const supa_amd_ew_desc* d, void* s) { return supa_amd_copy(d, s); }, "fill_");
    return self;
  }
  return fill_scalar(self, value.item());
}

at::Tensor& zero_(at::Tensor& self) { return fill_scalar(self, 0); }

at::Tensor& set_source_storage_offset(at::Tensor& self, c10::Storage source, int64_t offset, c10::IntArrayRef size,
                                      c10::IntArrayRef stride) {
  c10::TensorImpl* impl = self.unsafeGetTensorImpl();
  impl->set_storage_keep_dtype(std::move(source));
  impl->set_storage_offset(offset);
  impl->set_sizes_and_strides(size, stride);
  return self;
}

at::Tensor& set_source_storage(at::Tensor& self, c10::Storage source) {
  const int64_t n = (int64_t)(source.nbytes() / self.dtype().itemsize());
  return set_source_storage_offset(self, std::move(source), 0, {n}, {1});
}

at::Tensor& set_source_tensor(at::Tensor& self, const at::Tensor& src) {
  return set_source_storage_offset(self, src.storage(), src.storage_offset(), src.sizes(), src.strides());
}

at::Tensor& set_empty(at::Tensor& self) {
  c10::Storage st(c10::Storage::use_byte_size_t(), 0, allocator(), true);
  return set_source_storage_offset(self, st, 0, {0}, {1});
}

// ------------------------------------------------------------ binary ops
using Launch = EwLaunch;

Launch add_launch(const c10::Scalar& alpha, bool negate = false) {
  double a = 0.0;
  int64_t ia = 0;
  if (alpha.isBoolean()) {
    a = alpha.toBool() ? 1.0 : 0.0;
    ia = alpha.toBool() ? 1 : 0;
  } else if (alpha.isIntegral(false)) {
    ia = alpha.toLong();
    a = (double)ia;
  } else {
    a = alpha.toDouble();
    ia = (int64_t)a;
  }
  if (negate) {
    a = -a;
    ia = -ia;
  }
  return [a, ia](const supa_amd_ew_desc* d, void* s) { return supa_amd_add(d, a, ia, s); };
}

void check_alpha(c10::ScalarType common, const c10::Scalar& alpha) {
  TORCH_CHECK(!alpha.isBoolean() || common == at::kBool,
              "Boolean alpha only supported for Boolean results.");
  TORCH_CHECK(at::isFloatingType(common) || alpha.isIntegral(true),
              "For integral input tensors, argument alpha must not be a floating point number.");
}

at::Tensor binary(const at::Tensor& self, const at::Tensor& other, at::Tensor out, bool inplace,
                  const Launch& fn, const char* name, bool int_to_float = false, bool swap = false,
                  const c10::Scalar* alpha = nullptr) {
  c10::ScalarType common = at::result_type(self, other);
  if (int_to_float && at::isIntegralType(common, /*includeBool=*/true)) common = default_float();
  if (alpha) check_alpha(common, *alpha);
  std::vector<EwIn> ins = swap ? std::vector<EwIn>{EwIn::of(other), EwIn::of(self)}
                               : std::vector<EwIn>{EwIn::of(self), EwIn::of(other)};
  if (inplace) {
    check_cast(common, self, name);
    return ew_apply(self, self.scalar_type(), common, ins, fn, name);
  }
  if (out.defined()) {
    check_cast(common, out, name);
    return ew_apply(out, out.scalar_type(), common, ins, fn, name);
  }
  return ew_apply(at::Tensor(), common, common, ins, fn, name);
}

at::Tensor add_t(const at::Tensor& s, const at::Tensor& o, const c10::Scalar& a) {
  return binary(s, o, {}, false, add_launch(a), "add", false, false, &a);
}
at::Tensor& add_t_(at::Tensor& s, const at::Tensor& o, const c10::Scalar& a) {
  binary(s, o, {}, true, add_launch(a), "add_", false, false, &a);
  return s;
}
at::Tensor& add_out(const at::Tensor& s, const at::Tensor& o, const c10::Scalar& a, at::Tensor& out) {
  binary(s, o, out, false, add_launch(a), "add.out", false, false, &a);
  return out;
}
void check_sub(const at::Tensor& s, const at::Tensor& o) {
  TORCH_CHECK(s.scalar_type() != at::kBool || o.scalar_type() != at::kBool,
              "Subtraction, the `-` operator, with two bool tensors is not supported. Use the `^` or `logical_xor()` "
              "operator instead.");
}
at::Tensor sub_t(const at::Tensor& s, const at::Tensor& o, const c10::Scalar& a) {
  check_sub(s, o);
  return binary(s, o, {}, false, add_launch(a, true), "sub", false, false, &a);
}
at::Tensor& sub_t_(at::Tensor& s, const at::Tensor& o, const c10::Scalar& a) {
  check_sub(s, o);
  binary(s, o, {}, true, add_launch(a, true), "sub_", false, false, &a);
  return s;
}
at::Tensor& sub_out(const at::Tensor& s, const at::Tensor& o, const c10::Scalar& a, at::Tensor& out) {
  check_sub(s, o);
  binary(s, o, out, false, add_launch(a, true), "sub.out", false, false, &a);
  return out;
}
// rsub(self, other, alpha) = other - alpha * self
at::Tensor rsub_t(const at::Tensor& s, const at::Tensor& o, const c10::Scalar& a) {
  check_sub(s, o);
  return binary(s, o, {}, false, add_launch(a, true), "rsub", false, true, &a);
}

Launch mul_launch() {
  return [](const supa_amd_ew_desc* d, void* s) { return supa_amd_mul(d, s); };
}
at::Tensor mul_t(const at::Tensor& s, const at::Tensor& o) { return binary(s, o, {}, false, mul_launch(), "mul"); }
at::Tensor& mul_t_(at::Tensor& s, const at::Tensor& o) {
  binary(s, o, {}, true, mul_launch(), "mul_");
  return s;
}
at::Tensor& mul_out(const at::Tensor& s, const at::Tensor& o, at::Tensor& out) {
  binary(s, o, out, false, mul_launch(), "mul.out");
  return out;
}

int div_mode(std::optional<c10::string_view> mode) {
  if (!mode) return SUPA_AMD_DIV_TRUE;
  if (*mode == "trunc") return SUPA_AMD_DIV_TRUNC;
  if (*mode == "floor") return SUPA_AMD_DIV_FLOOR;
  TORCH_CHECK(false, "div expected rounding_mode to be one of None, 'trunc', or 'floor' but found '", *mode, "'");
}
Launch div_launch(int mode) {
  return [mode](const supa_amd_ew_desc* d, void* s) { return supa_amd_div(d, mode, s); };
}
at::Tensor div_tensor(const at::Tensor& s, const at::Tensor& o) {
  return binary(s, o, {}, false, div_launch(SUPA_AMD_DIV_TRUE), "div", true);
}
at::Tensor& div_tensor_(at::Tensor& s, const at::Tensor& o) {
  binary(s, o, {}, true, div_launch(SUPA_AMD_DIV_TRUE), "div_", true);
  return s;
}
at::Tensor& div_out(const at::Tensor& s, const at::Tensor& o, at::Tensor& out) {
  binary(s, o, out, false, div_launch(SUPA_AMD_DIV_TRUE), "div.out", true);
  return out;
}
at::Tensor div_tm(const at::Tensor& s, const at::Tensor& o, std::optional<c10::string_view> mode) {
  const int m = div_mode(mode);
  return binary(s, o, {}, false, div_launch(m), "div", m == SUPA_AMD_DIV_TRUE);
}
at::Tensor& div_tm_(at::Tensor& s, const at::Tensor& o, std::optional<c10::string_view> mode) {
  const int m = div_mode(mode);
  binary(s, o, {}, true, div_launch(m), "div_", m == SUPA_AMD_DIV_TRUE);
  return s;
}
at::Tensor& div_out_mode(const at::Tensor& s, const at::Tensor& o, std::optional<c10::string_view> mode,
                         at::Tensor& out) {
  const int m = div_mode(mode);
  binary(s, o, out, false, div_launch(m), "div.out_mode", m == SUPA_AMD_DIV_TRUE);
  return out;
}

// ------------------------------------------------- maximum / minimum / clamp
Launch minmax_launch(bool is_max) {
  return [is_max](const supa_amd_ew_desc* d, void* s) { return supa_amd_minmax(d, is_max ? 1 : 0, s); };
}
at::Tensor maximum_t(const at::Tensor& s, const at::Tensor& o) { return binary(s, o, {}, false, minmax_launch(true), "maximum"); }
at::Tensor& maximum_out(const at::Tensor& s, const at::Tensor& o, at::Tensor& out) {
  binary(s, o, out, false, minmax_launch(true), "maximum.out");
  return out;
}
at::Tensor minimum_t(const at::Tensor& s, const at::Tensor& o) { return binary(s, o, {}, false, minmax_launch(false), "minimum"); }
at::Tensor& minimum_out(const at::Tensor& s, const at::Tensor& o, at::Tensor& out) {
  binary(s, o, out, false, minmax_launch(false), "minimum.out");
  return out;
}

// clamp_min / clamp_max against a Scalar or a Tensor bound, with type
// promotion, as upstream's structured clamp_min / clamp_max.
at::Tensor clamp_bound(const at::Tensor& self, const c10::Scalar& bound, at::Tensor out, bool inplace, bool is_max_op,
                       const char* name) {
  TORCH_CHECK(self.scalar_type() != at::kBool, name, ": not implemented for 'Bool'");
  const c10::ScalarType common = at::result_type(self, bound);
  std::vector<EwIn> ins{EwIn::of(self), EwIn::num(bound)};
  const Launch fn = minmax_launch(is_max_op);
  if (inplace) {
    check_cast(common, self, name);
    return ew_apply(self, self.scalar_type(), common, ins, fn, name);
  }
  if (out.defined()) {
    check_cast(common, out, name);
    return ew_apply(out, out.scalar_type(), common, ins, fn, name);
  }
  return ew_apply(at::Tensor(), common, common, ins, fn, name);
}
// clamp_min(x, lo) = max(x, lo); clamp_max(x, hi) = min(x, hi)
at::Tensor clamp_min_s(const at::Tensor& s, const c10::Scalar& b) { return clamp_bound(s, b, {}, false, true, "clamp_min"); }
at::Tensor& clamp_min_s_(at::Tensor& s, const c10::Scalar& b) {
  clamp_bound(s, b, {}, true, true, "clamp_min_");
  return s;
}
at::Tensor& clamp_min_s_out(const at::Tensor& s, const c10::Scalar& b, at::Tensor& out) {
  clamp_bound(s, b, out, false, true, "clamp_min.out");
  return out;
}
at::Tensor clamp_max_s(const at::Tensor& s, const c10::Scalar& b) { return clamp_bound(s, b, {}, false, false, "clamp_max"); }
at::Tensor& clamp_max_s_(at::Tensor& s, const c10::Scalar& b) {
  clamp_bound(s, b, {}, true, false, "clamp_max_");
  return s;
}
at::Tensor& clamp_max_s_out(const at::Tensor& s, const c10::Scalar& b, at::Tensor& out) {
  clamp_bound(s, b, out, false, false, "clamp_max.out");
  return out;
}
at::Tensor clamp_min_t(const at::Tensor& s, const at::Tensor& b) { return binary(s, b, {}, false, minmax_launch(true), "clamp_min"); }
at::Tensor& clamp_min_t_(at::Tensor& s, const at::Tensor& b) {
  binary(s, b, {}, true, minmax_launch(true), "clamp_min_");
  return s;
}
at::Tensor& clamp_min_t_out(const at::Tensor& s, const at::Tensor& b, at::Tensor& out) {
  binary(s, b, out, false, minmax_launch(true), "clamp_min.Tensor_out");
  return out;
}
at::Tensor clamp_max_t(const at::Tensor& s, const at::Tensor& b) { return binary(s, b, {}, false, minmax_launch(false), "clamp_max"); }
at::Tensor& clamp_max_t_(at::Tensor& s, const at::Tensor& b) {
  binary(s, b, {}, true, minmax_launch(false), "clamp_max_");
  return s;
}
at::Tensor& clamp_max_t_out(const at::Tensor& s, const at::Tensor& b, at::Tensor& out) {
  binary(s, b, out, false, minmax_launch(false), "clamp_max.Tensor_out");
  return out;
}
// clamp(x, lo, hi) = min(max(x, lo), hi): a NaN x stays NaN, and lo > hi gives hi.
at::Tensor clamp_into(const at::Tensor& self, const std::optional<c10::Scalar>& lo,
                      const std::optional<c10::Scalar>& hi, at::Tensor dst, bool inplace, const char* name) {
  TORCH_CHECK(lo.has_value() || hi.has_value(), "torch.clamp: At least one of 'min' or 'max' must not be None");
  TORCH_CHECK(self.scalar_type() != at::kBool, name, ": not implemented for 'Bool'");
  at::native::ResultTypeState st = at::native::update_result_type_state(self, {});
  if (lo) st = at::native::update_result_type_state(*lo, st);
  if (hi) st = at::native::update_result_type_state(*hi, st);
  const c10::ScalarType common = at::native::result_type(st);
  if (dst.defined()) check_cast(common, dst, name);
  const c10::ScalarType out_dt = dst.defined() ? dst.scalar_type() : common;
  if (lo && hi) {
    at::Tensor tmp = ew_apply(at::Tensor(), common, common, {EwIn::of(self), EwIn::num(*lo)}, minmax_launch(true), name);
    return ew_apply(dst, out_dt, common, {EwIn::of(tmp), EwIn::num(*hi)}, minmax_launch(false), name);
  }
  return ew_apply(dst, out_dt, common, {EwIn::of(self), EwIn::num(lo ? *lo : *hi)}, minmax_launch(lo.has_value()),
                  name);
}
at::Tensor clamp_s(const at::Tensor& s, const std::optional<c10::Scalar>& lo, const std::optional<c10::Scalar>& hi) {
  return clamp_into(s, lo, hi, at::Tensor(), false, "clamp");
}
at::Tensor& clamp_s_(at::Tensor& s, const std::optional<c10::Scalar>& lo, const std::optional<c10::Scalar>& hi) {
  clamp_into(s, lo, hi, s, true, "clamp_");
  return s;
}
at::Tensor& clamp_s_out(const at::Tensor& s, const std::optional<c10::Scalar>& lo, const std::optional<c10::Scalar>& hi,
                        at::Tensor& out) {
  clamp_into(s, lo, hi, out, false, "clamp.out");
  return out;
}

// ---------------------------------------------- addcmul / addcdiv / lerp
Launch pointwise_launch(int op, const c10::Scalar& value) {
  double a = 0.0;
  int64_t ia = 0;
  if (value.isBoolean()) {
    a = value.toBool() ? 1.0 : 0.0;
    ia = value.toBool() ? 1 : 0;
  } else if (value.isIntegral(false)) {
    ia = value.toLong();
    a = (double)ia;
  } else {
    a = value.toDouble();
    ia = (int64_t)a;
  }
  return [op, a, ia](const supa_amd_ew_desc* d, void* s) { return supa_amd_pointwise(d, op, a, ia, s); };
}

at::Tensor ternary(const at::Tensor& self, const EwIn& b, const EwIn& c, c10::ScalarType common, at::Tensor out,
                   bool inplace, const Launch& fn, const char* name) {
  std::vector<EwIn> ins{EwIn::of(self), b, c};
  if (inplace) {
    check_cast(common, self, name);
    return ew_apply(self, self.scalar_type(), common, ins, fn, name);
  }
  if (out.defined()) {
    check_cast(common, out, name);
    return ew_apply(out, out.scalar_type(), common, ins, fn, name);
  }
  return ew_apply(at::Tensor(), common, common, ins, fn, name);
}

c10::ScalarType addc_common(const at::Tensor& self, const at::Tensor& t1, const at::Tensor& t2, bool div,
                            const char* name) {
  at::native::ResultTypeState st{};
  for (const at::Tensor* t : {&self, &t1, &t2}) st = at::native::update_result_type_state(*t, st);
  const c10::ScalarType common = at::native::result_type(st);
  if (div)
    TORCH_CHECK(!(at::isIntegralType(t1.scalar_type(), true) && at::isIntegralType(t2.scalar_type(), true)),
                "Integer division with addcdiv is no longer supported, and in a future release addcdiv will perform a "
                "true division of tensor1 and tensor2. The historic addcdiv behavior can be implemented as "
                "(input + value * torch.trunc(tensor1 / tensor2)).to(input.dtype) for integer inputs and as "
                "(input + value * tensor1 / tensor2) for float inputs. The future addcdiv behavior is just the "
                "latter implementation: (input + value * tensor1 / tensor2), for all dtypes.");
  (void)name;
  return common;
}

#define SUPA_ADDC(NAME, OP, DIV)                                                                                  \
  at::Tensor NAME(const at::Tensor& s, const at::Tensor& t1, const at::Tensor& t2, const c10::Scalar& v) {        \
    return ternary(s, EwIn::of(t1), EwIn::of(t2), addc_common(s, t1, t2, DIV, #NAME), {}, false,                   \
                   pointwise_launch(OP, v), #NAME);                                                                \
  }                                                                                                                \
  at::Tensor& NAME##_(at::Tensor& s, const at::Tensor& t1, const at::Tensor& t2, const c10::Scalar& v) {          \
    ternary(s, EwIn::of(t1), EwIn::of(t2), addc_common(s, t1, t2, DIV, #NAME), {}, true, pointwise_launch(OP, v),  \
            #NAME "_");                                                                                            \
    return s;                                                                                                      \
  }                                                                                                                \
  at::Tensor& NAME##_out(const at::Tensor& s, const at::Tensor& t1, const at::Tensor& t2, const c10::Scalar& v,   \
                         at::Tensor& out) {                                                                        \
    ternary(s, EwIn::of(t1), EwIn::of(t2), addc_common(s, t1, t2, DIV, #NAME), out, false,                         \
            pointwise_launch(OP, v), #NAME ".out");                                                                \
    return out;                                                                                                    \
  }
SUPA_ADDC(addcmul, SUPA_AMD_ADDCMUL, false)
SUPA_ADDC(addcdiv, SUPA_AMD_ADDCDIV, true)
#undef SUPA_ADDC

void lerp_checks(const at::Tensor& self, const at::Tensor& end, const at::Tensor* weight) {
  TORCH_CHECK(self.scalar_type() == end.scalar_type(), "expected dtype ", self.scalar_type(),
              " for `end` but got dtype ", end.scalar_type());
  if (weight)
    TORCH_CHECK(self.scalar_type() == weight->scalar_type(), "expected dtype ", self.scalar_type(),
                " for `weight` but got dtype ", weight->scalar_type());
  TORCH_CHECK(at::isFloatingType(self.scalar_type()), "lerp: expected a floating-point input, got ",
              self.scalar_type());
}
const Launch& lerp_launch() {
  static const Launch fn = [](const supa_amd_ew_desc* d, void* s) {
    return supa_amd_pointwise(d, SUPA_AMD_LERP, 0.0, 0, s);
  };
  return fn;
}
at::Tensor lerp_s(const at::Tensor& s, const at::Tensor& e, const c10::Scalar& w) {
  lerp_checks(s, e, nullptr);
  return ternary(s, EwIn::of(e), EwIn::num(w), s.scalar_type(), {}, false, lerp_launch(), "lerp");
}
at::Tensor& lerp_s_(at::Tensor& s, const at::Tensor& e, const c10::Scalar& w) {
  lerp_checks(s, e, nullptr);
  ternary(s, EwIn::of(e), EwIn::num(w), s.scalar_type(), {}, true, lerp_launch(), "lerp_");
  return s;
}
at::Tensor& lerp_s_out(const at::Tensor& s, const at::Tensor& e, const c10::Scalar& w, at::Tensor& out) {
  lerp_checks(s, e, nullptr);
  ternary(s, EwIn::of(e), EwIn::num(w), s.scalar_type(), out, false, lerp_launch(), "lerp.Scalar_out");
  return out;
}
at::Tensor lerp_t(const at::Tensor& s, const at::Tensor& e, const at::Tensor& w) {
  lerp_checks(s, e, &w);
  return ternary(s, EwIn::of(e), EwIn::of(w), s.scalar_type(), {}, false, lerp_launch(), "lerp");
}
at::Tensor& lerp_t_(at::Tensor& s, const at::Tensor& e, const at::Tensor& w) {
  lerp_checks(s, e, &w);
  ternary(s, EwIn::of(e), EwIn::of(w), s.scalar_type(), {}, true, lerp_launch(), "lerp_");
  return s;
}
at::Tensor& lerp_t_out(const at::Tensor& s, const at::Tensor& e, const at::Tensor& w, at::Tensor& out) {
  lerp_checks(s, e, &w);
  ternary(s, EwIn::of(e), EwIn::of(w), s.scalar_type(), out, false, lerp_launch(), "lerp.Tensor_out");
  return out;
}

// ------------------------------------------------------------------ cat
// cat (and stack, which upstream builds on it): each input is copied into
// its slice of the output by the copy kernel.  Upstream's rules: one result
// dtype over all inputs, legacy 1-D empty tensors skipped, every other input
// equal to the first in all dims but `dim`.
at::Tensor cat_supa(const at::ITensorListRef& tensors, int64_t dim) {
  const auto ts = tensors.materialize();
  TORCH_CHECK(!ts.empty(), "torch.cat(): expected a non-empty list of Tensors");
  auto legacy_empty = [](const at::Tensor& t) { return t.dim() == 1 && t.size(0) == 0; };
  const at::Tensor& first = ts[0].get();
  const c10::ScalarType dt = at::native::result_type(tensors);
  const at::Tensor* ref = nullptr;
  for (size_t i = 0; i < ts.size(); ++i) {
    const at::Tensor& t = ts[i].get();
    TORCH_CHECK(t.device() == first.device(), "Expected all tensors to be on the same device, but found at least "
                "two devices, ", first.device(), " and ", t.device(), "!");
    TORCH_CHECK(t.dim() > 0, "zero-dimensional tensor (at position ", i, ") cannot be concatenated");
    if (!ref && !legacy_empty(t)) ref = &t;
  }
  if (!ref) return at::empty({0}, first.options().dtype(dt));
  const int64_t d = at::maybe_wrap_dim(dim, ref->dim());
  std::vector<int64_t> size = ref->sizes().vec();
  int64_t total = 0;
  for (size_t i = 0; i < ts.size(); ++i) {
    const at::Tensor& t = ts[i].get();
    if (legacy_empty(t)) continue;
    TORCH_CHECK(t.dim() == ref->dim(), "Tensors must have same number of dimensions: got ", ref->dim(), " and ",
                t.dim());
    for (int64_t k = 0; k < t.dim(); ++k)
      TORCH_CHECK(k == d || t.size(k) == ref->size(k), "Sizes of tensors must match except in dimension ", d,
                  ". Expected size ", ref->size(k), " but got size ", t.size(k), " for tensor number ", i,
                  " in the list.");
    total += t.size(d);
  }
  size[d] = total;
  at::Tensor out = at::empty(size, first.options().dtype(dt));
  int64_t off = 0;
  for (const auto& r : ts) {
    const at::Tensor& t = r.get();
    if (legacy_empty(t) || t.size(d) == 0) continue;
    out.narrow(d, off, t.size(d)).copy_(t);
    off += t.size(d);
  }
  return out;
}

// ---------------------------------------------------------- activations
enum class UKind { FloatOnly, IntToFloat, Any };

at::Tensor unary(const at::Tensor& self, at::Tensor out, bool inplace, int op, UKind kind, const char* name) {
  c10::ScalarType common = self.scalar_type();
  if (kind == UKind::FloatOnly) {
    TORCH_CHECK(at::isFloatingType(common), name, ": \"", name, "\" not implemented for '", common, "'");
  } else if (kind == UKind::IntToFloat && at::isIntegralType(common, true)) {
    common = default_float();
  }
  const Launch fn = [op](const supa_amd_ew_desc* d, void* s) { return supa_amd_unary(d, op, s); };
  std::vector<EwIn> ins{EwIn::of(self)};
  if (inplace) {
    check_cast(common, self, name);
    return ew_apply(self, self.scalar_type(), common, ins, fn, name);
  }
  if (out.defined()) {
    check_cast(common, out, name);
    return ew_apply(out, out.scalar_type(), common, ins, fn, name);
  }
  return ew_apply(at::Tensor(), common, common, ins, fn, name);
}

at::Tensor unary_bwd(const at::Tensor& grad, const at::Tensor& x, at::Tensor out, int op, const char* name) {
  const c10::ScalarType common = at::result_type(grad, x);
  TORCH_CHECK(at::isFloatingType(common), name, ": not implemented for '", common, "'");
  const Launch fn = [op](const supa_amd_ew_desc* d, void* s) { return supa_amd_unary_backward(d, op, s); };
  std::vector<EwIn> ins{EwIn::of(grad), EwIn::of(x)};
  if (out.defined()) {
    check_cast(common, out, name);
    return ew_apply(out, out.scalar_type(), common, ins, fn, name);
  }
  return ew_apply(at::Tensor(), common, common, ins, fn, name);
}

int gelu_op(c10::string_view approximate) {
  const bool acc = accurate_gelu_enabled();
  if (approximate == "none") return acc ? SUPA_AMD_GELU_LOGERFC : SUPA_AMD_GELU;
  if (approximate == "tanh") return acc ? SUPA_AMD_GELU_TANH_LOGISTIC : SUPA_AMD_GELU_TANH;
  TORCH_CHECK(false, "approximate argument must be either none or tanh.");
}

at::Tensor gelu(const at::Tensor& s, c10::string_view a) { return unary(s, {}, false, gelu_op(a), UKind::FloatOnly, "gelu"); }
at::Tensor& gelu_(at::Tensor& s, c10::string_view a) {
  unary(s, {}, true, gelu_op(a), UKind::FloatOnly, "gelu_");
  return s;
}
at::Tensor& gelu_out(const at::Tensor& s, c10::string_view a, at::Tensor& out) {
  unary(s, out, false, gelu_op(a), UKind::FloatOnly, "gelu.out");
  return out;
}
at::Tensor gelu_backward(const at::Tensor& g, const at::Tensor& s, c10::string_view a) {
  return unary_bwd(g, s, {}, gelu_op(a), "gelu_backward");
}
at::Tensor& gelu_backward_out(const at::Tensor& g, const at::Tensor& s, c10::string_view a, at::Tensor& gi) {
  unary_bwd(g, s, gi, gelu_op(a), "gelu_backward.grad_input");
  return gi;
}

#define SUPA_UNARY(NAME, OP, KIND)                                                        \
  at::Tensor u_##NAME(const at::Tensor& s) { return unary(s, {}, false, OP, KIND, #NAME); } \
  at::Tensor& u_##NAME##_(at::Tensor& s) {                                                \
    unary(s, {}, true, OP, KIND, #NAME "_");                                              \
    return s;                                                                             \
  }                                                                                       \
  at::Tensor& u_##NAME##_out(const at::Tensor& s, at::Tensor& out) {                      \
    unary(s, out, false, OP, KIND, #NAME ".out");                                         \
    return out;                                                                           \
  }

SUPA_UNARY(silu, SUPA_AMD_SILU, UKind::FloatOnly)
SUPA_UNARY(sigmoid, SUPA_AMD_SIGMOID, UKind::IntToFloat)
SUPA_UNARY(tanh, SUPA_AMD_TANH, UKind::IntToFloat)
SUPA_UNARY(exp, SUPA_AMD_EXP, UKind::IntToFloat)
SUPA_UNARY(log, SUPA_AMD_LOG, UKind::IntToFloat)
SUPA_UNARY(erf, SUPA_AMD_ERF, UKind::IntToFloat)
SUPA_UNARY(neg, SUPA_AMD_NEG, UKind::Any)
SUPA_UNARY(reciprocal, SUPA_AMD_RECIPROCAL, UKind::IntToFloat)
SUPA_UNARY(abs, SUPA_AMD_ABS, UKind::Any)
SUPA_UNARY(sqrt, SUPA_AMD_SQRT, UKind::IntToFloat)
SUPA_UNARY(expm1, SUPA_AMD_EXPM1, UKind::IntToFloat)
SUPA_UNARY(log1p, SUPA_AMD_LOG1P, UKind::IntToFloat)
#undef SUPA_UNARY

at::Tensor relu(const at::Tensor& s) {
  TORCH_CHECK(s.scalar_type() != at::kBool, "Boolean inputs not supported for relu");
  return unary(s, {}, false, SUPA_AMD_RELU, UKind::Any, "relu");
}
at::Tensor& relu_(at::Tensor& s) {
  TORCH_CHECK(s.scalar_type() != at::kBool, "Boolean inputs not supported for relu");
  unary(s, {}, true, SUPA_AMD_RELU, UKind::Any, "relu_");
  return s;
}

#define SUPA_UNARY_BWD(NAME, OP)                                                             \
  at::Tensor NAME##_backward(const at::Tensor& g, const at::Tensor& x) {                     \
    return unary_bwd(g, x, {}, OP, #NAME "_backward");                                       \
  }                                                                                          \
  at::Tensor& NAME##_backward_out(const at::Tensor& g, const at::Tensor& x, at::Tensor& gi) { \
    unary_bwd(g, x, gi, OP, #NAME "_backward.grad_input");                                   \
    return gi;                                                                               \
  }
SUPA_UNARY_BWD(silu, SUPA_AMD_SILU)
SUPA_UNARY_BWD(sigmoid, SUPA_AMD_SIGMOID)
SUPA_UNARY_BWD(tanh, SUPA_AMD_TANH)
#undef SUPA_UNARY_BWD

// ------------------------------------------------ comparisons and selects
// eq/ne/lt/le/gt/ge: compared in the promoted dtype, a bool result (the out=
// tensor's dtype for .out, self's for the in-place forms).
Launch cmp_launch(int kind) {
  return [kind](const supa_amd_ew_desc* d, void* s) { return supa_amd_compare(d, kind, s); };
}
at::Tensor compare(const at::Tensor& self, const EwIn& other, c10::ScalarType common, at::Tensor out, bool inplace,
                   int kind, const char* name) {
  std::vector<EwIn> ins{EwIn::of(self), other};
  if (inplace) return ew_apply(self, self.scalar_type(), common, ins, cmp_launch(kind), name);
  if (out.defined()) return ew_apply(out, out.scalar_type(), common, ins, cmp_launch(kind), name);
  return ew_apply(at::Tensor(), at::kBool, common, ins, cmp_launch(kind), name);
}
#define SUPA_CMP(NAME, KIND)                                                                                      \
  at::Tensor NAME##_t(const at::Tensor& s, const at::Tensor& o) {                                                 \
    return compare(s, EwIn::of(o), at::result_type(s, o), {}, false, KIND, #NAME ".Tensor");                      \
  }                                                                                                               \
  at::Tensor& NAME##_t_(at::Tensor& s, const at::Tensor& o) {                                                     \
    compare(s, EwIn::of(o), at::result_type(s, o), {}, true, KIND, #NAME "_.Tensor");                             \
    return s;                                                                                                     \
  }                                                                                                               \
  at::Tensor& NAME##_t_out(const at::Tensor& s, const at::Tensor& o, at::Tensor& out) {                           \
    compare(s, EwIn::of(o), at::result_type(s, o), out, false, KIND, #NAME ".Tensor_out");                        \
    return out;                                                                                                   \
  }                                                                                                               \
  at::Tensor NAME##_s(const at::Tensor& s, const c10::Scalar& o) {                                                \
    return compare(s, EwIn::num(o), at::result_type(s, o), {}, false, KIND, #NAME ".Scalar");                     \
  }                                                                                                               \
  at::Tensor& NAME##_s_(at::Tensor& s, const c10::Scalar& o) {                                                    \
    compare(s, EwIn::num(o), at::result_type(s, o), {}, true, KIND, #NAME "_.Scalar");                            \
    return s;                                                                                                     \
  }                                                                                                               \
  at::Tensor& NAME##_s_out(const at::Tensor& s, const c10::Scalar& o, at::Tensor& out) {                          \
    compare(s, EwIn::num(o), at::result_type(s, o), out, false, KIND, #NAME ".Scalar_out");                       \
    return out;                                                                                                   \
  }
SUPA_CMP(eq, SUPA_AMD_CMP_EQ)
SUPA_CMP(ne, SUPA_AMD_CMP_NE)
SUPA_CMP(lt, SUPA_AMD_CMP_LT)
SUPA_CMP(le, SUPA_AMD_CMP_LE)
SUPA_CMP(gt, SUPA_AMD_CMP_GT)
SUPA_CMP(ge, SUPA_AMD_CMP_GE)
#undef SUPA_CMP

at::Tensor isnan_t(const at::Tensor& s) {
  const Launch fn = [](const supa_amd_ew_desc* d, void* st) { return supa_amd_isnan(d, st); };
  return ew_apply(at::Tensor(), at::kBool, s.scalar_type(), {EwIn::of(s)}, fn, "isnan");
}

Launch where_launch() {
  return [](const supa_amd_ew_desc* d, void* s) { return supa_amd_where(d, s); };
}
at::Tensor where_into(const at::Tensor& cond, const at::Tensor& a, const at::Tensor& b, at::Tensor out,
                      const char* name) {
  TORCH_CHECK(cond.scalar_type() == at::kBool,
              "where expected condition to be a boolean tensor, but got a tensor with dtype ", cond.scalar_type());
  const c10::ScalarType common = at::result_type(a, b);
  std::vector<EwIn> ins{EwIn::of(cond), EwIn::of(a), EwIn::of(b)};
  if (out.defined()) return ew_apply(out, out.scalar_type(), common, ins, where_launch(), name);
  return ew_apply(at::Tensor(), common, common, ins, where_launch(), name);
}
at::Tensor where_self(const at::Tensor& c, const at::Tensor& a, const at::Tensor& b) {
  return where_into(c, a, b, {}, "where.self");
}
at::Tensor& where_self_out(const at::Tensor& c, const at::Tensor& a, const at::Tensor& b, at::Tensor& out) {
  where_into(c, a, b, out, "where.self_out");
  return out;
}

// masked_fill_: self = mask ? value : self, the mask broadcast to self.
at::Tensor& masked_fill_s(at::Tensor& self, const at::Tensor& mask, const c10::Scalar& value) {
  TORCH_CHECK(mask.scalar_type() == at::kBool, "masked_fill_ only supports boolean masks, but got mask with dtype ",
              mask.scalar_type());
  TORCH_CHECK(self.device() == mask.device(), "expected self and mask to be on the same device, but got mask on ",
              mask.device(), " and self on ", self.device());
  ew_apply(self, self.scalar_type(), self.scalar_type(), {EwIn::of(mask), EwIn::num(value), EwIn::of(self)},
           where_launch(), "masked_fill_");
  return self;
}
at::Tensor& masked_fill_t(at::Tensor& self, const at::Tensor& mask, const at::Tensor& value) {
  TORCH_CHECK(value.dim() == 0, "masked_fill_ only supports a 0-dimensional value tensor, but got tensor with ",
              value.dim(), " dimension(s).");
  return masked_fill_s(self, mask, value.item());
}

// ------------------------------------------------ parameterised activations
// leaky_relu, elu, softplus, hardswish, hardsigmoid, mish, log_sigmoid,
// threshold and their backwards (hardtanh's forward is clamp), with
// upstream's argument checks (Activation.cpp).
at::Tensor act_apply(const at::Tensor& self, at::Tensor out, bool inplace, int act, double p0, double p1, double p2,
                     const char* name) {
  const c10::ScalarType common = self.scalar_type();
  if (act == SUPA_AMD_ACT_THRESHOLD) {
    TORCH_CHECK(common != at::kBool, name, ": \"", name, "\" not implemented for 'Bool'");
  } else {
    TORCH_CHECK(at::isFloatingType(common), name, ": \"", name, "\" not implemented for '", common, "'");
  }
  const Launch fn = [=](const supa_amd_ew_desc* d, void* s) { return supa_amd_activation(d, act, p0, p1, p2, s); };
  std::vector<EwIn> ins{EwIn::of(self)};
  if (inplace) return ew_apply(self, self.scalar_type(), common, ins, fn, name);
  if (out.defined()) {
    check_cast(common, out, name);
    return ew_apply(out, out.scalar_type(), common, ins, fn, name);
  }
  return ew_apply(at::Tensor(), common, common, ins, fn, name);
}

at::Tensor act_bwd_apply(const at::Tensor& grad, const at::Tensor& x, at::Tensor out, int act, double p0, double p1,
                         double p2, int flag, const char* name) {
  const c10::ScalarType common = at::result_type(grad, x);
  TORCH_CHECK(at::isFloatingType(common), name, ": not implemented for '", common, "'");
  const Launch fn = [=](const supa_amd_ew_desc* d, void* s) {
    return supa_amd_activation_backward(d, act, p0, p1, p2, flag, s);
  };
  std::vector<EwIn> ins{EwIn::of(grad), EwIn::of(x)};
  if (out.defined()) {
    check_cast(common, out, name);
    return ew_apply(out, out.scalar_type(), common, ins, fn, name);
  }
  return ew_apply(at::Tensor(), common, common, ins, fn, name);
}

double sd(const c10::Scalar& v) { return v.toDouble(); }

// leaky_relu
at::Tensor leaky_relu(const at::Tensor& s, const c10::Scalar& ns) {
  return act_apply(s, {}, false, SUPA_AMD_ACT_LEAKY_RELU, sd(ns), 0, 0, "leaky_relu");
}
at::Tensor& leaky_relu_(at::Tensor& s, const c10::Scalar& ns) {
  act_apply(s, {}, true, SUPA_AMD_ACT_LEAKY_RELU, sd(ns), 0, 0, "leaky_relu_");
  return s;
}
at::Tensor& leaky_relu_out(const at::Tensor& s, const c10::Scalar& ns, at::Tensor& out) {
  act_apply(s, out, false, SUPA_AMD_ACT_LEAKY_RELU, sd(ns), 0, 0, "leaky_relu.out");
  return out;
}
at::Tensor leaky_relu_bwd_into(const at::Tensor& g, const at::Tensor& s, const c10::Scalar& ns, bool self_is_result,
                               at::Tensor out, const char* name) {
  TORCH_CHECK(!self_is_result || ns.toDouble() >= 0.0,
              "In-place leakyReLu backward calculation is triggered with a negative slope which is not supported. "
              "This is caused by calling in-place forward function with a negative slope, please call out-of-place "
              "version instead. File an issue at https://github.com/pytorch/pytorch if you do require supporting "
              "in-place leakRelu backward calculation with negative slope");
  return act_bwd_apply(g, s, out, SUPA_AMD_ACT_LEAKY_RELU, sd(ns), 0, 0, 0, name);
}
at::Tensor leaky_relu_backward(const at::Tensor& g, const at::Tensor& s, const c10::Scalar& ns, bool r) {
  return leaky_relu_bwd_into(g, s, ns, r, {}, "leaky_relu_backward");
}
at::Tensor& leaky_relu_backward_out(const at::Tensor& g, const at::Tensor& s, const c10::Scalar& ns, bool r,
                                    at::Tensor& gi) {
  leaky_relu_bwd_into(g, s, ns, r, gi, "leaky_relu_backward.grad_input");
  return gi;
}

// hardtanh: the forward is clamp (upstream's hardtanh_out calls clamp_out)
at::Tensor hardtanh(const at::Tensor& s, const c10::Scalar& lo, const c10::Scalar& hi) {
  TORCH_CHECK(s.scalar_type() != at::kBool, "Bool inputs not supported for hardtanh");
  return at::clamp(s, lo, hi);
}
at::Tensor& hardtanh_(at::Tensor& s, const c10::Scalar& lo, const c10::Scalar& hi) {
  TORCH_CHECK(s.scalar_type() != at::kBool, "Bool inputs not supported for hardtanh");
  return at::clamp_(s, lo, hi);
}
at::Tensor& hardtanh_out(const at::Tensor& s, const c10::Scalar& lo, const c10::Scalar& hi, at::Tensor& out) {
  TORCH_CHECK(s.scalar_type() != at::kBool, "Bool inputs not supported for hardtanh");
  return at::clamp_out(out, s, lo, hi);
}
at::Tensor hardtanh_backward(const at::Tensor& g, const at::Tensor& s, const c10::Scalar& lo, const c10::Scalar& hi) {
  return act_bwd_apply(g, s, {}, SUPA_AMD_ACT_HARDTANH, sd(lo), sd(hi), 0, 0, "hardtanh_backward");
}
at::Tensor& hardtanh_backward_out(const at::Tensor& g, const at::Tensor& s, const c10::Scalar& lo,
                                  const c10::Scalar& hi, at::Tensor& gi) {
  act_bwd_apply(g, s, gi, SUPA_AMD_ACT_HARDTANH, sd(lo), sd(hi), 0, 0, "hardtanh_backward.grad_input");
  return gi;
}

// elu
at::Tensor elu(const at::Tensor& s, const c10::Scalar& a, const c10::Scalar& sc, const c10::Scalar& is) {
  return act_apply(s, {}, false, SUPA_AMD_ACT_ELU, sd(a), sd(sc), sd(is), "elu");
}
at::Tensor& elu_(at::Tensor& s, const c10::Scalar& a, const c10::Scalar& sc, const c10::Scalar& is) {
  act_apply(s, {}, true, SUPA_AMD_ACT_ELU, sd(a), sd(sc), sd(is), "elu_");
  return s;
}
at::Tensor& elu_out(const at::Tensor& s, const c10::Scalar& a, const c10::Scalar& sc, const c10::Scalar& is,
                    at::Tensor& out) {
  act_apply(s, out, false, SUPA_AMD_ACT_ELU, sd(a), sd(sc), sd(is), "elu.out");
  return out;
}
at::Tensor elu_bwd_into(const at::Tensor& g, const c10::Scalar& a, const c10::Scalar& sc, const c10::Scalar& is,
                        bool is_result, const at::Tensor& x, at::Tensor out, const char* name) {
  if (is_result) {
    TORCH_CHECK(a.toDouble() >= 0.0, "In-place elu backward calculation is triggered with a negative slope which "
                "is not supported. This is caused by calling in-place forward function with a negative slope, "
                "please call out-of-place version instead.");
  }
  return act_bwd_apply(g, x, out, SUPA_AMD_ACT_ELU, sd(a), sd(sc), sd(is), is_result ? 1 : 0, name);
}
at::Tensor elu_backward(const at::Tensor& g, const c10::Scalar& a, const c10::Scalar& sc, const c10::Scalar& is,
                        bool r, const at::Tensor& x) {
  return elu_bwd_into(g, a, sc, is, r, x, {}, "elu_backward");
}
at::Tensor& elu_backward_out(const at::Tensor& g, const c10::Scalar& a, const c10::Scalar& sc, const c10::Scalar& is,
                             bool r, const at::Tensor& x, at::Tensor& gi) {
  elu_bwd_into(g, a, sc, is, r, x, gi, "elu_backward.grad_input");
  return gi;
}

// softplus
at::Tensor softplus(const at::Tensor& s, const c10::Scalar& b, const c10::Scalar& th) {
  return act_apply(s, {}, false, SUPA_AMD_ACT_SOFTPLUS, sd(b), sd(th), 0, "softplus");
}
at::Tensor& softplus_out(const at::Tensor& s, const c10::Scalar& b, const c10::Scalar& th, at::Tensor& out) {
  act_apply(s, out, false, SUPA_AMD_ACT_SOFTPLUS, sd(b), sd(th), 0, "softplus.out");
  return out;
}
at::Tensor softplus_backward(const at::Tensor& g, const at::Tensor& s, const c10::Scalar& b, const c10::Scalar& th) {
  return act_bwd_apply(g, s, {}, SUPA_AMD_ACT_SOFTPLUS, sd(b), sd(th), 0, 0, "softplus_backward");
}
at::Tensor& softplus_backward_out(const at::Tensor& g, const at::Tensor& s, const c10::Scalar& b,
                                  const c10::Scalar& th, at::Tensor& gi) {
  act_bwd_apply(g, s, gi, SUPA_AMD_ACT_SOFTPLUS, sd(b), sd(th), 0, 0, "softplus_backward.grad_input");
  return gi;
}

// hardswish, hardsigmoid, mish: no parameters
#define SUPA_ACT0(NAME, ACT)                                                                       \
  at::Tensor NAME(const at::Tensor& s) { return act_apply(s, {}, false, ACT, 0, 0, 0, #NAME); }     \
  at::Tensor& NAME##_(at::Tensor& s) {                                                             \
    act_apply(s, {}, true, ACT, 0, 0, 0, #NAME "_");                                               \
    return s;                                                                                      \
  }                                                                                                \
  at::Tensor& NAME##_out(const at::Tensor& s, at::Tensor& out) {                                   \
    act_apply(s, out, false, ACT, 0, 0, 0, #NAME ".out");                                          \
    return out;                                                                                    \
  }                                                                                                \
  at::Tensor NAME##_backward(const at::Tensor& g, const at::Tensor& s) {                           \
    return act_bwd_apply(g, s, {}, ACT, 0, 0, 0, 0, #NAME "_backward");                            \
  }                                                                                                \
  at::Tensor& NAME##_backward_out(const at::Tensor& g, const at::Tensor& s, at::Tensor& gi) {      \
    act_bwd_apply(g, s, gi, ACT, 0, 0, 0, 0, #NAME "_backward.grad_input");                        \
    return gi;                                                                                     \
  }
SUPA_ACT0(hardswish, SUPA_AMD_ACT_HARDSWISH)
SUPA_ACT0(hardsigmoid, SUPA_AMD_ACT_HARDSIGMOID)
SUPA_ACT0(mish, SUPA_AMD_ACT_MISH)
#undef SUPA_ACT0

// log_sigmoid: the forward's buffer is empty, as on upstream's CUDA backend
std::tuple<at::Tensor, at::Tensor> log_sigmoid_forward(const at::Tensor& s) {
  at::Tensor out = act_apply(s, {}, false, SUPA_AMD_ACT_LOG_SIGMOID, 0, 0, 0, "log_sigmoid_forward");
  return {out, at::empty({0}, s.options())};
}
std::tuple<at::Tensor&, at::Tensor&> log_sigmoid_forward_out(const at::Tensor& s, at::Tensor& out, at::Tensor& buf) {
  act_apply(s, out, false, SUPA_AMD_ACT_LOG_SIGMOID, 0, 0, 0, "log_sigmoid_forward.output");
  at::native::resize_output(buf, {0});
  return {out, buf};
}
at::Tensor log_sigmoid_backward(const at::Tensor& g, const at::Tensor& s, const at::Tensor& /*buffer*/) {
  return act_bwd_apply(g, s, {}, SUPA_AMD_ACT_LOG_SIGMOID, 0, 0, 0, 0, "log_sigmoid_backward");
}
at::Tensor& log_sigmoid_backward_out(const at::Tensor& g, const at::Tensor& s, const at::Tensor& /*buffer*/,
                                     at::Tensor& gi) {
  act_bwd_apply(g, s, gi, SUPA_AMD_ACT_LOG_SIGMOID, 0, 0, 0, 0, "log_sigmoid_backward.grad_input");
  return gi;
}

// threshold (relu's backward is threshold_backward(grad, result, 0))
at::Tensor threshold(const at::Tensor& s, const c10::Scalar& th, const c10::Scalar& v) {
  return act_apply(s, {}, false, SUPA_AMD_ACT_THRESHOLD, sd(th), sd(v), 0, "threshold");
}
at::Tensor& threshold_(at::Tensor& s, const c10::Scalar& th, const c10::Scalar& v) {
  act_apply(s, {}, true, SUPA_AMD_ACT_THRESHOLD, sd(th), sd(v), 0, "threshold_");
  return s;
}
at::Tensor& threshold_out(const at::Tensor& s, const c10::Scalar& th, const c10::Scalar& v, at::Tensor& out) {
  act_apply(s, out, false, SUPA_AMD_ACT_THRESHOLD, sd(th), sd(v), 0, "threshold.out");
  return out;
}
at::Tensor threshold_backward(const at::Tensor& g, const at::Tensor& s, const c10::Scalar& th) {
  return act_bwd_apply(g, s, {}, SUPA_AMD_ACT_THRESHOLD, sd(th), 0, 0, 0, "threshold_backward");
}
at::Tensor& threshold_backward_out(const at::Tensor& g, const at::Tensor& s, const c10::Scalar& th, at::Tensor& gi) {
  act_bwd_apply(g, s, gi, SUPA_AMD_ACT_THRESHOLD, sd(th), 0, 0, 0, "threshold_backward.grad_input");
  return gi;
}

// hardshrink / softshrink and their shared backward (upstream Activation.cpp:
// softshrink refuses a negative lambda)
void check_softshrink(const c10::Scalar& l) {
  TORCH_CHECK(sd(l) >= 0, "lambda must be greater or equal to 0, but found to be ", sd(l), ".");
}
at::Tensor hardshrink(const at::Tensor& s, const c10::Scalar& l) {
  return act_apply(s, {}, false, SUPA_AMD_ACT_HARDSHRINK, sd(l), 0, 0, "hardshrink");
}
at::Tensor& hardshrink_out(const at::Tensor& s, const c10::Scalar& l, at::Tensor& out) {
  act_apply(s, out, false, SUPA_AMD_ACT_HARDSHRINK, sd(l), 0, 0, "hardshrink.out");
  return out;
}
at::Tensor hardshrink_backward(const at::Tensor& g, const at::Tensor& s, const c10::Scalar& l) {
  return act_bwd_apply(g, s, {}, SUPA_AMD_ACT_HARDSHRINK, sd(l), 0, 0, 0, "hardshrink_backward");
}
at::Tensor& hardshrink_backward_out(const at::Tensor& g, const at::Tensor& s, const c10::Scalar& l, at::Tensor& gi) {
  act_bwd_apply(g, s, gi, SUPA_AMD_ACT_HARDSHRINK, sd(l), 0, 0, 0, "hardshrink_backward.grad_input");
  return gi;
}
at::Tensor softshrink(const at::Tensor& s, const c10::Scalar& l) {
  check_softshrink(l);
  return act_apply(s, {}, false, SUPA_AMD_ACT_SOFTSHRINK, sd(l), 0, 0, "softshrink");
}
at::Tensor& softshrink_out(const at::Tensor& s, const c10::Scalar& l, at::Tensor& out) {
  check_softshrink(l);
  act_apply(s, out, false, SUPA_AMD_ACT_SOFTSHRINK, sd(l), 0, 0, "softshrink.out");
  return out;
}
at::Tensor softshrink_backward(const at::Tensor& g, const at::Tensor& s, const c10::Scalar& l) {
  return act_bwd_apply(g, s, {}, SUPA_AMD_ACT_SOFTSHRINK, sd(l), 0, 0, 0, "softshrink_backward");
}
at::Tensor& softshrink_backward_out(const at::Tensor& g, const at::Tensor& s, const c10::Scalar& l, at::Tensor& gi) {
  act_bwd_apply(g, s, gi, SUPA_AMD_ACT_SOFTSHRINK, sd(l), 0, 0, 0, "softshrink_backward.grad_input");
  return gi;
}

// glu: the two halves along dim as strided views of the input, one binary
// launch (upstream GatedLinearUnit.cpp's checks and halving).
int64_t glu_dim(const at::Tensor& self, int64_t dim) {
  TORCH_CHECK(self.dim() > 0, "glu does not support scalars because halving size must be even");
  const int64_t wd = at::maybe_wrap_dim(dim, self.dim());
  TORCH_CHECK(self.size(wd) % 2 == 0, "Halving dimension must be even, but dimension ", wd, " is size ",
              self.size(wd));
  return wd;
}
at::Tensor glu_into(const at::Tensor& self, int64_t dim, at::Tensor out, const char* name) {
  const int64_t wd = glu_dim(self, dim);
  const int64_t h = self.size(wd) / 2;
  const c10::ScalarType common = self.scalar_type();
  TORCH_CHECK(at::isFloatingType(common), name, ": \"glu\" not implemented for '", common, "'");
  const Launch fn = [](const supa_amd_ew_desc* d, void* s) { return supa_amd_glu(d, s); };
  std::vector<EwIn> ins{EwIn::of(self.narrow(wd, 0, h)), EwIn::of(self.narrow(wd, h, h))};
  if (out.defined()) {
    check_cast(common, out, name);
    return ew_apply(out, out.scalar_type(), common, ins, fn, name);
  }
  return ew_apply(at::Tensor(), common, common, ins, fn, name);
}
at::Tensor glu(const at::Tensor& self, int64_t dim) { return glu_into(self, dim, {}, "glu"); }
at::Tensor& glu_out(const at::Tensor& self, int64_t dim, at::Tensor& out) {
  glu_into(self, dim, out, "glu.out");
  return out;
}
// glu_backward writes each half of grad_input (sized as the input) through a
// strided view of it, one launch per half.
at::Tensor& glu_backward_into(const at::Tensor& g, const at::Tensor& self, int64_t dim, at::Tensor& gi,
                              const char* name) {
  const int64_t wd = glu_dim(self, dim);
  const int64_t h = self.size(wd) / 2;
  const c10::ScalarType common = at::result_type(g, self);
  TORCH_CHECK(at::isFloatingType(common), name, ": not implemented for '", common, "'");
  at::native::resize_output(gi, self.sizes());
  const at::Tensor a = self.narrow(wd, 0, h), b = self.narrow(wd, h, h);
  at::Tensor ga = gi.narrow(wd, 0, h), gb = gi.narrow(wd, h, h);
  ew_apply(ga, gi.scalar_type(), common, {EwIn::of(b), EwIn::of(g)},
           [](const supa_amd_ew_desc* d, void* s) { return supa_amd_glu_backward(d, 0, s); }, name);
  ew_apply(gb, gi.scalar_type(), common, {EwIn::of(a), EwIn::of(b), EwIn::of(g)},
           [](const supa_amd_ew_desc* d, void* s) { return supa_amd_glu_backward(d, 1, s); }, name);
  return gi;
}
at::Tensor glu_backward(const at::Tensor& g, const at::Tensor& self, int64_t dim) {
  at::Tensor gi = at::empty_like(self);
  return glu_backward_into(g, self, dim, gi, "glu_backward");
}
at::Tensor& glu_backward_out(const at::Tensor& g, const at::Tensor& self, int64_t dim, at::Tensor& gi) {
  return glu_backward_into(g, self, dim, gi, "glu_backward.grad_input");
}

// prelu's kernels (upstream _prelu_kernel / _prelu_kernel_backward; the
// composite prelu has already shaped the weight to broadcast over self).  The
// backward's weight gradient is elementwise, at the broadcast shape.
at::Tensor prelu_kernel(const at::Tensor& self, const at::Tensor& weight) {
  const c10::ScalarType common = at::result_type(self, weight);
  TORCH_CHECK(at::isFloatingType(common), "_prelu_kernel: \"prelu\" not implemented for '", common, "'");
  return ew_apply(at::Tensor(), self.scalar_type(), common, {EwIn::of(self), EwIn::of(weight)},
                  [](const supa_amd_ew_desc* d, void* s) { return supa_amd_prelu(d, s); }, "_prelu_kernel");
}
std::tuple<at::Tensor, at::Tensor> prelu_kernel_backward(const at::Tensor& g, const at::Tensor& self,
                                                         const at::Tensor& weight) {
  const c10::ScalarType common = c10::promoteTypes(at::result_type(self, weight), g.scalar_type());
  TORCH_CHECK(at::isFloatingType(common), "_prelu_kernel_backward: not implemented for '", common, "'");
  at::Tensor gs = ew_apply(at::Tensor(), self.scalar_type(), common,
                           {EwIn::of(self), EwIn::of(weight), EwIn::of(g)},
                           [](const supa_amd_ew_desc* d, void* s) { return supa_amd_prelu_backward(d, 0, s); },
                           "_prelu_kernel_backward");
  at::Tensor gw = ew_apply(at::Tensor(), weight.scalar_type(), common,
                           {EwIn::of(self), EwIn::of(g)},
                           [](const supa_amd_ew_desc* d, void* s) { return supa_amd_prelu_backward(d, 1, s); },
                           "_prelu_kernel_backward");
  return {gs, gw};
}

}  // namespace
}  // namespace supa

TORCH_LIBRARY_IMPL(aten, PrivateUse1, m) {
  using namespace supa;
  // tensor plumbing
  m.impl("empty.memory_format", TORCH_FN(empty_memory_format));
  m.impl("empty_strided", TORCH_FN(empty_strided));
  m.impl("as_strided", TORCH_FN(at::native::as_strided_tensorimpl));
  m.impl("view", TORCH_FN(at::native::view));
  m.impl("_reshape_alias", TORCH_FN(at::native::_reshape_alias));
  m.impl("resize_", TORCH_FN(resize_));
  m.impl("_copy_from", TORCH_FN(copy_from));
  m.impl("_copy_from_and_resize", TORCH_FN(copy_from_and_resize));
  m.impl("_local_scalar_dense", TORCH_FN(local_scalar_dense));
  m.impl("equal", TORCH_FN(equal));
  m.impl("eye.out", TORCH_FN(eye_out));
  m.impl("scatter_.value", TORCH_FN(scatter_value_));
  m.impl("scatter.value", TORCH_FN(scatter_value));
  m.impl("scatter.value_out", TORCH_FN(scatter_value_out));
  m.impl("eye.m_out", TORCH_FN(eye_m_out));
  m.impl("fill_.Scalar", TORCH_FN(fill_scalar));
  m.impl("fill_.Tensor", TORCH_FN(fill_tensor));
  m.impl("zero_", TORCH_FN(zero_));
  m.impl("set_.source_Storage", TORCH_FN(set_source_storage));
  m.impl("set_.source_Storage_storage_offset", TORCH_FN(set_source_storage_offset));
  m.impl("set_.source_Tensor", TORCH_FN(set_source_tensor));
  m.impl("set_", TORCH_FN(set_empty));
  // binary
  m.impl("add.Tensor", TORCH_FN(add_t));
  m.impl("add_.Tensor", TORCH_FN(add_t_));
  m.impl("add.out", TORCH_FN(add_out));
  m.impl("sub.Tensor", TORCH_FN(sub_t));
  m.impl("sub_.Tensor", TORCH_FN(sub_t_));
  m.impl("sub.out", TORCH_FN(sub_out));
  m.impl("rsub.Tensor", TORCH_FN(rsub_t));
  m.impl("mul.Tensor", TORCH_FN(mul_t));
  m.impl("mul_.Tensor", TORCH_FN(mul_t_));
  m.impl("mul.out", TORCH_FN(mul_out));
  m.impl("div.Tensor", TORCH_FN(div_tensor));
  m.impl("div_.Tensor", TORCH_FN(div_tensor_));
  m.impl("div.out", TORCH_FN(div_out));
  m.impl("div.Tensor_mode", TORCH_FN(div_tm));
  m.impl("div_.Tensor_mode", TORCH_FN(div_tm_));
  m.impl("div.out_mode", TORCH_FN(div_out_mode));
  // activations
  m.impl("cat", TORCH_FN(cat_supa));
  m.impl("maximum", TORCH_FN(maximum_t));
  m.impl("maximum.out", TORCH_FN(maximum_out));
  m.impl("minimum", TORCH_FN(minimum_t));
  m.impl("minimum.out", TORCH_FN(minimum_out));
  m.impl("clamp_min", TORCH_FN(clamp_min_s));
  m.impl("clamp_min_", TORCH_FN(clamp_min_s_));
  m.impl("clamp_min.out", TORCH_FN(clamp_min_s_out));
  m.impl("clamp_min.Tensor", TORCH_FN(clamp_min_t));
  m.impl("clamp_min_.Tensor", TORCH_FN(clamp_min_t_));
  m.impl("clamp_min.Tensor_out", TORCH_FN(clamp_min_t_out));
  m.impl("clamp_max", TORCH_FN(clamp_max_s));
  m.impl("clamp_max_", TORCH_FN(clamp_max_s_));
  m.impl("clamp_max.out", TORCH_FN(clamp_max_s_out));
  m.impl("clamp_max.Tensor", TORCH_FN(clamp_max_t));
  m.impl("clamp_max_.Tensor", TORCH_FN(clamp_max_t_));
  m.impl("clamp_max.Tensor_out", TORCH_FN(clamp_max_t_out));
  m.impl("clamp", TORCH_FN(clamp_s));
  m.impl("clamp_", TORCH_FN(clamp_s_));
  m.impl("clamp.out", TORCH_FN(clamp_s_out));
  m.impl("addcmul", TORCH_FN(addcmul));
  m.impl("addcmul_", TORCH_FN(addcmul_));
  m.impl("addcmul.out", TORCH_FN(addcmul_out));
  m.impl("addcdiv", TORCH_FN(addcdiv));
  m.impl("addcdiv_", TORCH_FN(addcdiv_));
  m.impl("addcdiv.out", TORCH_FN(addcdiv_out));
  m.impl("lerp.Scalar", TORCH_FN(lerp_s));
  m.impl("lerp_.Scalar", TORCH_FN(lerp_s_));
  m.impl("lerp.Scalar_out", TORCH_FN(lerp_s_out));
  m.impl("lerp.Tensor", TORCH_FN(lerp_t));
  m.impl("lerp_.Tensor", TORCH_FN(lerp_t_));
  m.impl("lerp.Tensor_out", TORCH_FN(lerp_t_out));
#define SUPA_REG_CMP(NAME)                                    \
  m.impl(#NAME ".Tensor", TORCH_FN(NAME##_t));                \
  m.impl(#NAME "_.Tensor", TORCH_FN(NAME##_t_));              \
  m.impl(#NAME ".Tensor_out", TORCH_FN(NAME##_t_out));        \
  m.impl(#NAME ".Scalar", TORCH_FN(NAME##_s));                \
  m.impl(#NAME "_.Scalar", TORCH_FN(NAME##_s_));              \
  m.impl(#NAME ".Scalar_out", TORCH_FN(NAME##_s_out));
  SUPA_REG_CMP(eq)
  SUPA_REG_CMP(ne)
  SUPA_REG_CMP(lt)
  SUPA_REG_CMP(le)
  SUPA_REG_CMP(gt)
  SUPA_REG_CMP(ge)
#undef SUPA_REG_CMP
  m.impl("isnan", TORCH_FN(isnan_t));
  m.impl("where.self", TORCH_FN(where_self));
  m.impl("where.self_out", TORCH_FN(where_self_out));
  m.impl("masked_fill_.Scalar", TORCH_FN(masked_fill_s));
  m.impl("masked_fill_.Tensor", TORCH_FN(masked_fill_t));
  m.impl("leaky_relu", TORCH_FN(leaky_relu));
  m.impl("leaky_relu_", TORCH_FN(leaky_relu_));
  m.impl("leaky_relu.out", TORCH_FN(leaky_relu_out));
  m.impl("leaky_relu_backward", TORCH_FN(leaky_relu_backward));
  m.impl("leaky_relu_backward.grad_input", TORCH_FN(leaky_relu_backward_out));
  m.impl("hardtanh", TORCH_FN(hardtanh));
  m.impl("hardtanh_", TORCH_FN(hardtanh_));
  m.impl("hardtanh.out", TORCH_FN(hardtanh_out));
  m.impl("hardtanh_backward", TORCH_FN(hardtanh_backward));
  m.impl("hardtanh_backward.grad_input", TORCH_FN(hardtanh_backward_out));
  m.impl("elu", TORCH_FN(elu));
  m.impl("elu_", TORCH_FN(elu_));
  m.impl("elu.out", TORCH_FN(elu_out));
  m.impl("elu_backward", TORCH_FN(elu_backward));
  m.impl("elu_backward.grad_input", TORCH_FN(elu_backward_out));
  m.impl("softplus", TORCH_FN(softplus));
  m.impl("softplus.out", TORCH_FN(softplus_out));
  m.impl("softplus_backward", TORCH_FN(softplus_backward));
  m.impl("softplus_backward.grad_input", TORCH_FN(softplus_backward_out));
  m.impl("hardswish", TORCH_FN(hardswish));
  m.impl("hardswish_", TORCH_FN(hardswish_));
  m.impl("hardswish.out", TORCH_FN(hardswish_out));
  m.impl("hardswish_backward", TORCH_FN(hardswish_backward));
  m.impl("hardsigmoid", TORCH_FN(hardsigmoid));
  m.impl("hardsigmoid_", TORCH_FN(hardsigmoid_));
  m.impl("hardsigmoid.out", TORCH_FN(hardsigmoid_out));
  m.impl("hardsigmoid_backward", TORCH_FN(hardsigmoid_backward));
  m.impl("hardsigmoid_backward.grad_input", TORCH_FN(hardsigmoid_backward_out));
  m.impl("mish", TORCH_FN(mish));
  m.impl("mish_", TORCH_FN(mish_));
  m.impl("mish.out", TORCH_FN(mish_out));
  m.impl("mish_backward", TORCH_FN(mish_backward));
  m.impl("log_sigmoid_forward", TORCH_FN(log_sigmoid_forward));
  m.impl("log_sigmoid_forward.output", TORCH_FN(log_sigmoid_forward_out));
  m.impl("log_sigmoid_backward", TORCH_FN(log_sigmoid_backward));
  m.impl("log_sigmoid_backward.grad_input", TORCH_FN(log_sigmoid_backward_out));
  m.impl("threshold", TORCH_FN(threshold));
  m.impl("threshold_", TORCH_FN(threshold_));
  m.impl("threshold.out", TORCH_FN(threshold_out));
  m.impl("threshold_backward", TORCH_FN(threshold_backward));
  m.impl("threshold_backward.grad_input", TORCH_FN(threshold_backward_out));
  m.impl("hardshrink", TORCH_FN(hardshrink));
  m.impl("hardshrink.out", TORCH_FN(hardshrink_out));
  m.impl("hardshrink_backward", TORCH_FN(hardshrink_backward));
  m.impl("hardshrink_backward.grad_input", TORCH_FN(hardshrink_backward_out));
  m.impl("softshrink", TORCH_FN(softshrink));
  m.impl("softshrink.out", TORCH_FN(softshrink_out));
  m.impl("softshrink_backward", TORCH_FN(softshrink_backward));
  m.impl("softshrink_backward.grad_input", TORCH_FN(softshrink_backward_out));
  m.impl("glu", TORCH_FN(glu));
  m.impl("glu.out", TORCH_FN(glu_out));
  m.impl("glu_backward", TORCH_FN(glu_backward));
  m.impl("glu_backward.grad_input", TORCH_FN(glu_backward_out));
  m.impl("_prelu_kernel", TORCH_FN(prelu_kernel));
  m.impl("_prelu_kernel_backward", TORCH_FN(prelu_kernel_backward));
  m.impl("gelu", TORCH_FN(gelu));
  m.impl("gelu_", TORCH_FN(gelu_));
  m.impl("gelu.out", TORCH_FN(gelu_out));
  m.impl("gelu_backward", TORCH_FN(gelu_backward));
  m.impl("gelu_backward.grad_input", TORCH_FN(gelu_backward_out));
  m.impl("silu", TORCH_FN(u_silu));
  m.impl("silu_", TORCH_FN(u_silu_));
  m.impl("silu.out", TORCH_FN(u_silu_out));
  m.impl("silu_backward", TORCH_FN(silu_backward));
  m.impl("silu_backward.grad_input", TORCH_FN(silu_backward_out));
  m.impl("sigmoid", TORCH_FN(u_sigmoid));
  m.impl("sigmoid_", TORCH_FN(u_sigmoid_));
  m.impl("sigmoid.out", TORCH_FN(u_sigmoid_out));
  m.impl("sigmoid_backward", TORCH_FN(sigmoid_backward));
  m.impl("sigmoid_backward.grad_input", TORCH_FN(sigmoid_backward_out));
  m.impl("tanh", TORCH_FN(u_tanh));
  m.impl("tanh_", TORCH_FN(u_tanh_));
  m.impl("tanh.out", TORCH_FN(u_tanh_out));
  m.impl("tanh_backward", TORCH_FN(tanh_backward));
  m.impl("tanh_backward.grad_input", TORCH_FN(tanh_backward_out));
  m.impl("exp", TORCH_FN(u_exp));
  m.impl("exp_", TORCH_FN(u_exp_));
  m.impl("exp.out", TORCH_FN(u_exp_out));
  m.impl("log", TORCH_FN(u_log));
  m.impl("log_", TORCH_FN(u_log_));
  m.impl("log.out", TORCH_FN(u_log_out));
  m.impl("erf", TORCH_FN(u_erf));
  m.impl("erf_", TORCH_FN(u_erf_));
  m.impl("erf.out", TORCH_FN(u_erf_out));
  m.impl("neg", TORCH_FN(u_neg));
  m.impl("neg_", TORCH_FN(u_neg_));
  m.impl("neg.out", TORCH_FN(u_neg_out));
  m.impl("reciprocal", TORCH_FN(u_reciprocal));
  m.impl("reciprocal_", TORCH_FN(u_reciprocal_));
  m.impl("reciprocal.out", TORCH_FN(u_reciprocal_out));
  m.impl("abs", TORCH_FN(u_abs));
  m.impl("abs_", TORCH_FN(u_abs_));
  m.impl("abs.out", TORCH_FN(u_abs_out));
  m.impl("sqrt", TORCH_FN(u_sqrt));
  m.impl("sqrt_", TORCH_FN(u_sqrt_));
  m.impl("sqrt.out", TORCH_FN(u_sqrt_out));
  m.impl("expm1", TORCH_FN(u_expm1));
  m.impl("expm1_", TORCH_FN(u_expm1_));
  m.impl("expm1.out", TORCH_FN(u_expm1_out));
  m.impl("log1p", TORCH_FN(u_log1p));
  m.impl("log1p_", TORCH_FN(u_log1p_));
  m.impl("log1p.out", TORCH_FN(u_log1p_out));
  m.impl("relu", TORCH_FN(relu));
  m.impl("relu_", TORCH_FN(relu_));
}
