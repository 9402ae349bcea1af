// Host helper that runs one elementwise op through the planner and the C ABI.
#pragma once

#include <functional>
#include <vector>

#include "common.h"
#include "planner.h"

namespace supa {

// One input of an elementwise op: a supa tensor, or a host scalar (a Python
// number, or a 0-dim CPU tensor, both lifted into the kernel's functor).
struct EwIn {
  at::Tensor t;           // defined for tensor inputs
  bool scalar = false;    // host scalar
  c10::Scalar value;      // its value
  static EwIn of(const at::Tensor& x);  // 0-dim CPU tensors become scalars
  static EwIn num(const c10::Scalar& s) {
    EwIn e;
    e.scalar = true;
    e.value = s;
    return e;
  }
};

using EwLaunch = std::function<int(const supa_amd_ew_desc*, void*)>;

// Runs `launch` over (out, inputs...).  `out` may be undefined: it is then
// allocated with out_dtype and the planner's layout.  A defined `out` whose
// shape differs from the broadcast shape is resized.  common_dtype is the
// dtype inputs are converted to before the op.  Returns out.
at::Tensor ew_apply(at::Tensor out, c10::ScalarType out_dtype, c10::ScalarType common_dtype,
                    const std::vector<EwIn>& ins, const EwLaunch& launch, const char* name);

// The device every supa tensor among `ts` lives on (checks they agree and
// that no other non-scalar CPU tensor is mixed in).
c10::DeviceIndex common_device(const std::vector<const at::Tensor*>& ts, const char* name);

}  // namespace supa
