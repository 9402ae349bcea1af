// Python module torch_supa._C: device queries, streams and events, allocator
// statistics, CPU fallback control, and the planner (exposed for the CPU test
// tier).  The reference's counterpart is torch_supa/csrc/InitSupaBindings.cpp
// plus csrc/supa/Module.cpp:1133-1162 (device/stream/memory APIs).
#include <pybind11/pybind11.h>
#include <pybind11/stl.h>
#include <torch/extension.h>

#include "common.h"
#include "generator.h"
#include "planner.h"

namespace py = pybind11;

namespace {

py::dict memory_stats(int dev) {
  const supa::AllocatorStats s = supa::allocator_stats(static_cast<c10::DeviceIndex>(dev));
  py::dict d;
  d["allocated_bytes"] = s.allocated;
  d["reserved_bytes"] = s.reserved;
  d["peak_allocated_bytes"] = s.peak_allocated;
  d["num_allocs"] = s.num_allocs;
  d["num_device_mallocs"] = s.num_device_mallocs;
  d["num_frees"] = s.num_frees;
  d["num_ooms_retried"] = s.num_ooms_retried;
  d["peak_reserved_bytes"] = s.peak_reserved;
  d["pending_blocks"] = s.pending_blocks;
  return d;
}

// hipGetDeviceProperties, the fields torch.supa.get_device_properties shows.
py::dict device_properties(int dev) {
  hipDeviceProp_t p;
  SUPA_HIP_CHECK(hipGetDeviceProperties(&p, dev));
  py::dict d;
  d["name"] = std::string(p.name);
  d["total_memory"] = (int64_t)p.totalGlobalMem;
  d["major"] = p.major;
  d["minor"] = p.minor;
  d["multi_processor_count"] = p.multiProcessorCount;
  d["gcn_arch_name"] = std::string(p.gcnArchName);
  d["l2_cache_size"] = (int64_t)p.l2CacheSize;
  d["uuid"] = py::bytes(reinterpret_cast<const char*>(p.uuid.bytes), 16);
  return d;
}

// (free, total) device memory in bytes, as hipMemGetInfo reports them.
py::tuple mem_get_info(int dev) {
  const auto prev = supa::current_device();
  if (dev != prev) supa::set_device(static_cast<c10::DeviceIndex>(dev));
  size_t free_b = 0, total_b = 0;
  const hipError_t rc = hipMemGetInfo(&free_b, &total_b);
  if (dev != prev) supa::set_device(prev);
  SUPA_HIP_CHECK(rc);
  return py::make_tuple((int64_t)free_b, (int64_t)total_b);
}

// Planner entry for tests: operands are dicts {sizes, strides, is_output,
// allocate, scalar}.
py::dict plan(const py::list& ops) {
  std::vector<supa::PlanOperand> v;
  for (const auto& h : ops) {
    const py::dict d = h.cast<py::dict>();
    supa::PlanOperand p;
    if (d.contains("sizes")) p.sizes = d["sizes"].cast<std::vector<int64_t>>();
    if (d.contains("strides")) p.strides = d["strides"].cast<std::vector<int64_t>>();
    p.is_output = d.contains("is_output") && d["is_output"].cast<bool>();
    p.allocate = d.contains("allocate") && d["allocate"].cast<bool>();
    p.scalar = d.contains("scalar") && d["scalar"].cast<bool>();
    v.push_back(p);
  }
  supa::Plan p;
  try {
    p = supa::make_plan(v);
  } catch (const std::invalid_argument& e) {
    throw py::value_error(e.what());
  }
  py::dict r;
  r["shape"] = p.shape;
  r["out_strides"] = p.out_strides;
  r["it_sizes"] = p.it_sizes;
  r["it_strides"] = p.it_strides;
  r["numel"] = p.numel;
  return r;
}

uintptr_t event_create() {
  hipEvent_t e;
  SUPA_HIP_CHECK(hipEventCreate(&e));
  return reinterpret_cast<uintptr_t>(e);
}
// Records on stream `id` of device `dev` (-1: the current device / stream).
void event_record(uintptr_t e, int dev, int64_t id) {
  const auto d = dev < 0 ? supa::current_device() : static_cast<c10::DeviceIndex>(dev);
  const hipStream_t st = id < 0 ? supa::current_stream(d) : supa::stream_handle(d, id);
  SUPA_HIP_CHECK(hipEventRecord(reinterpret_cast<hipEvent_t>(e), st));
}
// Stream `id` of device `dev` waits for the event.
void event_wait(uintptr_t e, int dev, int64_t id) {
  const auto d = dev < 0 ? supa::current_device() : static_cast<c10::DeviceIndex>(dev);
  const hipStream_t st = id < 0 ? supa::current_stream(d) : supa::stream_handle(d, id);
  SUPA_HIP_CHECK(hipStreamWaitEvent(st, reinterpret_cast<hipEvent_t>(e), 0));
}
bool event_query(uintptr_t e) {
  const hipError_t rc = hipEventQuery(reinterpret_cast<hipEvent_t>(e));
  if (rc == hipErrorNotReady) {
    (void)hipGetLastError();
    return false;
  }
  SUPA_HIP_CHECK(rc);
  return true;
}
int64_t current_stream_id(int dev) { return supa::current_stream_obj(static_cast<c10::DeviceIndex>(dev)).id(); }
int64_t set_current_stream_id(int dev, int64_t id) {
  const c10::Stream s(c10::Stream::UNSAFE, c10::Device(supa::kSupa, static_cast<c10::DeviceIndex>(dev)), id);
  return supa::exchange_stream(s).id();
}
int64_t pool_stream_id(int dev) { return supa::pool_stream(static_cast<c10::DeviceIndex>(dev)).id(); }
uintptr_t stream_ptr(int dev, int64_t id) {
  return reinterpret_cast<uintptr_t>(supa::stream_handle(static_cast<c10::DeviceIndex>(dev), id));
}
void stream_synchronize(int dev, int64_t id) {
  SUPA_HIP_CHECK(hipStreamSynchronize(supa::stream_handle(static_cast<c10::DeviceIndex>(dev), id)));
}
bool stream_query(int dev, int64_t id) {
  const hipError_t rc = hipStreamQuery(supa::stream_handle(static_cast<c10::DeviceIndex>(dev), id));
  if (rc == hipErrorNotReady) {
    (void)hipGetLastError();
    return false;
  }
  SUPA_HIP_CHECK(rc);
  return true;
}
void event_synchronize(uintptr_t e) { SUPA_HIP_CHECK(hipEventSynchronize(reinterpret_cast<hipEvent_t>(e))); }
float event_elapsed_ms(uintptr_t a, uintptr_t b) {
  float ms = 0.f;
  SUPA_HIP_CHECK(hipEventElapsedTime(&ms, reinterpret_cast<hipEvent_t>(a), reinterpret_cast<hipEvent_t>(b)));
  return ms;
}
void event_destroy(uintptr_t e) { (void)hipEventDestroy(reinterpret_cast<hipEvent_t>(e)); }

// Device-to-device byte copy on the supa stream (used by harnesses that build
// inputs with another device API in the same process).
void memcpy_d2d(uintptr_t dst, uintptr_t src, int64_t nbytes) {
  SUPA_HIP_CHECK(hipMemcpyAsync(reinterpret_cast<void*>(dst), reinterpret_cast<const void*>(src), (size_t)nbytes,
                                hipMemcpyDeviceToDevice, supa::current_stream(supa::current_device())));
}

// The device's default Philox generator, for torch.supa's seeding API.
supa::SupaGenerator* gen_of(int dev) {
  return supa::default_generator(static_cast<c10::DeviceIndex>(dev)).get<supa::SupaGenerator>();
}
void rng_manual_seed(int dev, uint64_t seed) {
  supa::SupaGenerator* g = gen_of(dev);
  std::lock_guard<std::mutex> lock(g->mutex_);
  g->set_current_seed(seed);
}
uint64_t rng_seed(int dev) {
  supa::SupaGenerator* g = gen_of(dev);
  std::lock_guard<std::mutex> lock(g->mutex_);
  return g->seed();
}
uint64_t rng_initial_seed(int dev) { return gen_of(dev)->current_seed(); }
at::Tensor rng_get_state(int dev) {
  supa::SupaGenerator* g = gen_of(dev);
  std::lock_guard<std::mutex> lock(g->mutex_);
  return at::Tensor::wrap_tensor_impl(g->get_state());
}
void rng_set_state(int dev, const at::Tensor& st) {
  supa::SupaGenerator* g = gen_of(dev);
  std::lock_guard<std::mutex> lock(g->mutex_);
  g->set_state(*st.unsafeGetTensorImpl());
}

}  // namespace

PYBIND11_MODULE(_C, m) {
  m.doc() = "MI355X PrivateUse1 backend for the elementwise + loss operator path";
  m.def("device_count", []() { return (int)supa::device_count(); });
  m.def("current_device", []() { return (int)supa::current_device(); });
  m.def("set_device", [](int d) { supa::set_device(static_cast<c10::DeviceIndex>(d)); });
  m.def("synchronize", [](int d) { supa::synchronize(static_cast<c10::DeviceIndex>(d)); });
  m.def("memory_stats", &memory_stats);
  m.def("reset_peak_memory_stats", [](int d) { supa::allocator_reset_peak(static_cast<c10::DeviceIndex>(d)); });
  m.def("empty_cache", []() { supa::allocator_empty_cache(); });
  m.def("empty_host_cache", []() { supa::pinned_empty_cache(); });
  m.def("set_cpu_fallback_enabled", &supa::set_cpu_fallback_enabled);
  m.def("cpu_fallback_enabled", &supa::cpu_fallback_enabled);
  m.def("set_fused_cross_entropy_mode", &supa::set_fused_cross_entropy_mode);
  m.def("fused_cross_entropy_mode", &supa::fused_cross_entropy_mode);
  m.def("set_fused_bce_backward_enabled", &supa::set_fused_bce_backward_enabled);
  m.def("fused_bce_backward_enabled", &supa::fused_bce_backward_enabled);
  m.def("set_accurate_gelu_enabled", &supa::set_accurate_gelu_enabled);
  m.def("accurate_gelu_enabled", &supa::accurate_gelu_enabled);
  m.def("fallback_counts", &supa::fallback_counts);
  m.def("reset_fallback_counts", &supa::reset_fallback_counts);
  m.def("plan", &plan);
  m.def("abi_version", []() { return supa_amd_abi_version(); });
  m.def("event_create", &event_create);
  m.def("event_record", &event_record, py::arg("event"), py::arg("device") = -1, py::arg("stream_id") = -1);
  m.def("event_wait", &event_wait, py::arg("event"), py::arg("device") = -1, py::arg("stream_id") = -1);
  m.def("event_query", &event_query);
  m.def("current_stream_id", &current_stream_id);
  m.def("set_current_stream_id", &set_current_stream_id);
  m.def("pool_stream_id", &pool_stream_id);
  m.def("stream_ptr", &stream_ptr);
  m.def("stream_synchronize", &stream_synchronize);
  m.def("stream_query", &stream_query);
  m.def("record_stream", [](const at::Tensor& t, int dev, int64_t id) {
    const c10::Stream s(c10::Stream::UNSAFE, c10::Device(supa::kSupa, static_cast<c10::DeviceIndex>(dev)), id);
    supa::allocator_record_stream(t.storage().data_ptr().get(), s);
  });
  m.def("inject_oom", [](int n) { supa::allocator_inject_oom(n); });
  m.def("device_properties", &device_properties);
  m.def("mem_get_info", &mem_get_info);
  m.def("raw_alloc", [](size_t nbytes, int dev, uintptr_t stream) {
    return reinterpret_cast<uintptr_t>(
        supa::allocator_raw_alloc(nbytes, static_cast<c10::DeviceIndex>(dev), reinterpret_cast<hipStream_t>(stream)));
  });
  m.def("raw_delete", [](uintptr_t p) { supa::allocator_raw_delete(reinterpret_cast<void*>(p)); });
  m.def("set_memory_fraction", [](double f, int dev) {
    supa::allocator_set_memory_fraction(f, static_cast<c10::DeviceIndex>(dev));
  });
  m.def("get_memory_fraction",
        [](int dev) { return supa::allocator_get_memory_fraction(static_cast<c10::DeviceIndex>(dev)); });
  m.def("event_synchronize", &event_synchronize);
  m.def("event_elapsed_ms", &event_elapsed_ms);
  m.def("event_destroy", &event_destroy);
  m.def("memcpy_d2d", &memcpy_d2d);
  m.def("rng_manual_seed", &rng_manual_seed);
  m.def("rng_seed", &rng_seed);
  m.def("rng_initial_seed", &rng_initial_seed);
  m.def("rng_get_state", &rng_get_state);
  m.def("rng_set_state", &rng_set_state);
}
