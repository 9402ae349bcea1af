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
// SUPA_LAUNCH_BLOCKING / CUDA_LAUNCH_BLOCKING: check_status synchronises after each launch.
bool launch_blocking();

// ------------------------------------------------------------- runtime
c10::DeviceIndex device_count() noexcept;
c10::DeviceIndex current_device();
void set_device(c10::DeviceIndex d);
// Streams: per device a non-blocking default stream (id 0) and a pool of 32
// (ids 1..32); the current stream is thread-local per device.
hipStream_t current_stream(c10::DeviceIndex d);  // the current stream's handle
hipStream_t stream_handle(c10::DeviceIndex d, c10::StreamId id);
c10::Stream current_stream_obj(c10::DeviceIndex d);
c10::Stream default_stream_obj(c10::DeviceIndex d);
c10::Stream pool_stream(c10::DeviceIndex d);        // round-robin over the pool
c10::Stream exchange_stream(const c10::Stream& s);  // makes s current on its device, returns the previous
void synchronize(c10::DeviceIndex d);               // every stream of device d
// Host <-> device copies ordered after the current stream's work; they return
// once the copy is complete.
void memcpy_h2d(void* dst, const void* src, size_t n, c10::DeviceIndex d);
void memcpy_d2h(void* dst, const void* src, size_t n, c10::DeviceIndex d);
c10::Allocator* allocator();

struct AllocatorStats {
  int64_t allocated = 0;
  int64_t reserved = 0;
  int64_t peak_allocated = 0;
  int64_t peak_reserved = 0;
  int64_t num_allocs = 0;
  int64_t num_device_mallocs = 0;
  int64_t num_frees = 0;
  int64_t num_ooms_retried = 0;  // hipMalloc failures retried after releasing the cache
  int64_t pending_blocks = 0;    // freed blocks waiting for other streams' events
};
AllocatorStats allocator_stats(c10::DeviceIndex d);
void allocator_reset_peak(c10::DeviceIndex d);
void allocator_empty_cache();
// the cached pinned host blocks back to the driver
void pinned_empty_cache();
// caching_allocator_alloc / _delete: a raw block of the allocator for stream
// st of device d (nullptr for 0 bytes), and its release.
void* allocator_raw_alloc(size_t nbytes, c10::DeviceIndex d, hipStream_t st);
void allocator_raw_delete(void* p);
// set_ / get_per_process_memory_fraction: at most fraction x total memory
// reserved on device d.
void allocator_set_memory_fraction(double fraction, c10::DeviceIndex d);
double allocator_get_memory_fraction(c10::DeviceIndex d);
// record_stream: the block holding ptr is also used on stream s.
void allocator_record_stream(void* ptr, const c10::Stream& s);
// Test hook: the next n device allocations fail as out of memory.
void allocator_inject_oom(int n);

// Per-device state owned by the runtime, allocated and zeroed once: the
// device error flag, which kernels only ever set (to report an out-of-range
// target) and the host clears when it reads it.  Reduction workspaces are not
// here: they come from the caching allocator per call, ordered on the
// calling stream.
// Device-side error flags: one int32 per stream of a device (the default
// stream and the pool), in one 256-byte block.  A kernel that finds a bad
// index (an nll_loss target, a scatter_ index) sets the flag of the stream it
// runs on, so a flag is read only once that stream's work is done.
struct DeviceScratch {
  int32_t* error_flags = nullptr;  // [stream id], ids 0..32
};
const DeviceScratch& device_scratch(c10::DeviceIndex d);
// The flag of device d's current stream, for the kernels launched on it.
int32_t* stream_error_flag(c10::DeviceIndex d);
// Raises (and clears) a pending device-side error of device d's current
// stream, e.g. an out-of-range nll_loss target.  Called after the current
// stream has synchronised (device-to-host copies, .item(), launch-blocking
// mode); an error of a kernel on another stream is reported once that stream
// has been synchronised (or by torch.supa.synchronize()).
void check_device_errors(c10::DeviceIndex d);

// CPU fallback bookkeeping (the fallback never runs for an op this library
// registers; tests assert that with these counters).
void set_cpu_fallback_enabled(bool on);
bool cpu_fallback_enabled();
// Fused cross-entropy routing: -1 the reference's (float32 logits fused,
// bfloat16 / float16 through the log_softmax + nll_loss decomposition), 0 no
// dtype fused, 1 every floating dtype fused.  Env SUPA_AMD_FUSED_CE=0 / 1.
void set_fused_cross_entropy_mode(int mode);
int fused_cross_entropy_mode();
// One-pass BCE-with-logits gradient (default on, env SUPA_AMD_FUSED_BCE=0 turns it off).
void set_fused_bce_backward_enabled(bool on);
bool fused_bce_backward_enabled();
// Cancellation-free gelu forms instead of the reference's (x/2)(1 + erf) and
// (x/2)(1 + tanh) (opt-in; default off, env SUPA_AMD_ACCURATE_GELU=1 turns it on).
void set_accurate_gelu_enabled(bool on);
bool accurate_gelu_enabled();
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
