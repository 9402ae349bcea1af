// The supa device's Philox generator (seed + per-call offset).
#pragma once

#include <ATen/core/Generator.h>
#include <c10/core/GeneratorImpl.h>

#include <optional>
#include <utility>

#include "common.h"

namespace supa {

// torch's default seed for device generators (the CUDA generator's
// default_rng_seed_val), so an unseeded process starts from a fixed stream.
constexpr uint64_t kDefaultSeed = 67280421310721ull;

struct SupaGenerator final : public c10::GeneratorImpl {
  explicit SupaGenerator(c10::DeviceIndex d, uint64_t seed = kDefaultSeed);
  void set_current_seed(uint64_t seed) override;
  void set_offset(uint64_t offset) override;
  uint64_t get_offset() const override;
  uint64_t current_seed() const override;
  uint64_t seed() override;
  void set_state(const c10::TensorImpl& new_state) override;
  c10::intrusive_ptr<c10::TensorImpl> get_state() const override;
  static c10::DeviceType device_type() { return kSupa; }
  // (seed, offset) for one random op; moves the offset on by one.
  std::pair<uint64_t, uint64_t> next_call();

 private:
  SupaGenerator* clone_impl() const override;
  uint64_t seed_;
  uint64_t offset_ = 0;
};

const at::Generator& default_generator(c10::DeviceIndex d);
at::Generator new_generator(c10::DeviceIndex d);
// (seed, offset) of `gen`, or of device d's default generator.
std::pair<uint64_t, uint64_t> philox_inputs(const std::optional<at::Generator>& gen, c10::DeviceIndex d);

}  // namespace supa
