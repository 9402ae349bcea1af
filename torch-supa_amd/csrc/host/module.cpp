// Python module torch_supa._C: device queries, allocator statistics, CPU
// fallback control, timing events, and the planner (exposed for the CPU test
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
  return d;
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
void event_record(uintptr_t e) {
  SUPA_HIP_CHECK(hipEventRecord(reinterpret_cast<hipEvent_t>(e), supa::current_stream(supa::current_device())));
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
  m.def("set_cpu_fallback_enabled", &supa::set_cpu_fallback_enabled);
  m.def("cpu_fallback_enabled", &supa::cpu_fallback_enabled);
  m.def("set_fused_cross_entropy_enabled", &supa::set_fused_cross_entropy_enabled);
  m.def("fused_cross_entropy_enabled", &supa::fused_cross_entropy_enabled);
  m.def("set_fused_bce_backward_enabled", &supa::set_fused_bce_backward_enabled);
  m.def("fused_bce_backward_enabled", &supa::fused_bce_backward_enabled);
  m.def("fallback_counts", &supa::fallback_counts);
  m.def("reset_fallback_counts", &supa::reset_fallback_counts);
  m.def("plan", &plan);
  m.def("abi_version", []() { return supa_amd_abi_version(); });
  m.def("event_create", &event_create);
  m.def("event_record", &event_record);
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
