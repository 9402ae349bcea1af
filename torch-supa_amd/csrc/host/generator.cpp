// Per-device random-number generator of the supa device: a Philox key (the
// seed) and a call offset.  Every random op takes (seed, offset) and moves
// the offset on by one, so consecutive calls draw from disjoint counter
// ranges of the same stream (the kernels index the counter by element).
// The counterpart of the reference's SUPAGeneratorImpl
// (torch_supa/csrc/aten/SUPAGeneratorImpl.h), reached through the
// PrivateUse1 hooks' getDefaultGenerator / getNewGenerator.
#include "generator.h"

#include <ATen/core/Generator.h>
#include <ATen/Utils.h>
#include <c10/core/GeneratorImpl.h>
#include <c10/core/TensorImpl.h>

#include <mutex>
#include <vector>

namespace supa {

SupaGenerator::SupaGenerator(c10::DeviceIndex d, uint64_t seed)
    : c10::GeneratorImpl(c10::Device(kSupa, d), c10::DispatchKeySet(c10::DispatchKey::PrivateUse1)), seed_(seed) {}

void SupaGenerator::set_current_seed(uint64_t seed) {
  seed_ = seed;
  offset_ = 0;
}
void SupaGenerator::set_offset(uint64_t offset) { offset_ = offset; }
uint64_t SupaGenerator::get_offset() const { return offset_; }
uint64_t SupaGenerator::current_seed() const { return seed_; }
uint64_t SupaGenerator::seed() {
  const uint64_t s = c10::detail::getNonDeterministicRandom();
  set_current_seed(s);
  return s;
}

// State: a 16-byte CPU uint8 tensor, the seed then the offset (little endian),
// the layout of the reference's SUPAGeneratorImpl::get_state / set_state
// (torch_supa/csrc/aten/SUPAGeneratorImpl.cpp:250-290).  The offset here
// counts calls (the counter's high half), not Philox draws per thread.
c10::intrusive_ptr<c10::TensorImpl> SupaGenerator::get_state() const {
  at::Tensor st = at::empty({16}, at::TensorOptions().dtype(at::kByte).device(at::kCPU));
  uint8_t* p = st.data_ptr<uint8_t>();
  for (int i = 0; i < 8; ++i) {
    p[i] = (uint8_t)(seed_ >> (8 * i));
    p[8 + i] = (uint8_t)(offset_ >> (8 * i));
  }
  return st.getIntrusivePtr();
}
void SupaGenerator::set_state(const c10::TensorImpl& new_state) {
  at::detail::check_rng_state(new_state);
  TORCH_CHECK(new_state.numel() == 16, "supa generator state must hold 16 bytes, got ", new_state.numel());
  const uint8_t* p = new_state.data_dtype_initialized<uint8_t>();
  uint64_t s = 0, o = 0;
  for (int i = 0; i < 8; ++i) {
    s |= (uint64_t)p[i] << (8 * i);
    o |= (uint64_t)p[8 + i] << (8 * i);
  }
  seed_ = s;
  offset_ = o;
}

std::pair<uint64_t, uint64_t> SupaGenerator::next_call() {
  const std::pair<uint64_t, uint64_t> r{seed_, offset_};
  offset_ += 1;
  return r;
}

SupaGenerator* SupaGenerator::clone_impl() const {
  auto* g = new SupaGenerator(device().index(), seed_);
  g->offset_ = offset_;
  return g;
}

namespace {
constexpr int kGenDevices = 64;
std::once_flag g_gen_once[kGenDevices];
at::Generator g_default_gens[kGenDevices];
}  // namespace

const at::Generator& default_generator(c10::DeviceIndex d) {
  if (d < 0) d = current_device();
  TORCH_CHECK(d < kGenDevices, "supa: device index out of range");
  std::call_once(g_gen_once[d], [d] { g_default_gens[d] = at::make_generator<SupaGenerator>(d); });
  return g_default_gens[d];
}

at::Generator new_generator(c10::DeviceIndex d) {
  return at::make_generator<SupaGenerator>(d < 0 ? current_device() : d);
}

std::pair<uint64_t, uint64_t> philox_inputs(const std::optional<at::Generator>& gen, c10::DeviceIndex d) {
  SupaGenerator* g = at::get_generator_or_default<SupaGenerator>(gen, default_generator(d));
  std::lock_guard<std::mutex> lock(g->mutex_);
  return g->next_call();
}

}  // namespace supa
