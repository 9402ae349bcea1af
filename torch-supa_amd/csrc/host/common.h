// Shared declarations of the host layer (PrivateUse1 runtime + operator
// registrations).  The host layer owns tensors, allocation and the dispatcher
// contract; every device computation goes through the C ABI in supa_amd.h.
#pragma once

#include <ATen/ATen.h>
#include <ATen/core/dispatch/Dispatcher.h>
#include <c10/core/Device.h>
#include <hip/hip_runtime_api.h>

#include <string>

#include "supa_amd.h"

namespace supa {

constexpr c10::DeviceType kSupa = c10::DeviceType::PrivateUse1;

#define SUPA_HIP_CHECK(expr)                                                              \
  do {                                                                                    \
    const hipError_t err__ = (expr);                                                      \
    TORCH_CHECK(err__ == hipSuccess, "HIP error ", hipGetErrorName(err__), ": ",        \
                hipGetErrorString(err__), " at ", __FILE__, ":", __LINE__);               \
  } while (0)

// Turns a non-zero C-ABI status into a c10::Error naming the op.
void check_status(int status, const char* what);

// ------------------------------------------------------------- runtime
c10::DeviceIndex device_count() noexcept;
c10::DeviceIndex current_device();
void set_device(c10::DeviceIndex d);
// The stream kernels are enqueued on for device d (the legacy default stream).
hipStream_t current_stream(c10::DeviceIndex d);
void synchronize(c10::DeviceIndex d);
c10::Allocator* allocator();

struct AllocatorStats {
  int64_t allocated = 0;
  int64_t reserved = 0;
  int64_t peak_allocated = 0;
  int64_t num_allocs = 0;
  int64_t num_device_mallocs = 0;
  int64_t num_frees = 0;
};
AllocatorStats allocator_stats(c10::DeviceIndex d);
void allocator_reset_peak(c10::DeviceIndex d);
void allocator_empty_cache();

// Per-device scratch owned by the runtime: allocated and zeroed once, never
// returned to the caching allocator.  Holds the reduction workspace (whose
// counter every reduction leaves at zero) and the device error flag.
struct DeviceScratch {
  void* reduce_ws = nullptr;
  int64_t reduce_ws_bytes = 0;
  int32_t* error_flag = nullptr;
};
const DeviceScratch& device_scratch(c10::DeviceIndex d);
// Raises (and clears) a pending device-side error, e.g. an out-of-range
// nll_loss target.  Called at every host synchronisation point.
void check_device_errors(c10::DeviceIndex d);

// CPU fallback bookkeeping (the fallback never runs for an op this library
// registers; tests assert that with these counters).
void set_cpu_fallback_enabled(bool on);
bool cpu_fallback_enabled();
// Fused cross-entropy (opt-in; default off, env SUPA_AMD_FUSED_CE=1 turns it on).
void set_fused_cross_entropy_enabled(bool on);
bool fused_cross_entropy_enabled();
// One-pass BCE-with-logits gradient (default on, env SUPA_AMD_FUSED_BCE=0 turns it off).
void set_fused_bce_backward_enabled(bool on);
bool fused_bce_backward_enabled();
std::vector<std::pair<std::string, int64_t>> fallback_counts();
void reset_fallback_counts();
// The boxed CPU fallback itself (counted; an error while disabled), for
// registered kernels that hand a case they do not cover over to it.
void supa_cpu_fallback(const c10::OperatorHandle& op, std::vector<c10::IValue>* stack);

// ------------------------------------------------------------ helpers
inline int32_t dtype_code(c10::ScalarType t) { return static_cast<int32_t>(t); }
bool dtype_supported(c10::ScalarType t);

// An empty tensor on the supa device with explicit strides.
at::Tensor empty_strided_supa(c10::IntArrayRef size, c10::IntArrayRef stride, c10::ScalarType dtype,
                              c10::DeviceIndex device);
at::Tensor empty_supa(c10::IntArrayRef size, c10::ScalarType dtype, c10::DeviceIndex device,
                      c10::MemoryFormat fmt = c10::MemoryFormat::Contiguous);

}  // namespace supa
