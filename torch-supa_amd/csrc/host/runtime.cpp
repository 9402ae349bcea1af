// PrivateUse1 runtime for MI355X: caching allocator, device guard, hooks and
// the boxed CPU fallback.
//
// Replaces, at the scale this path needs, the reference's runtime core
// (torch_supa/csrc/core/supa/): SUPACachingAllocator (REGISTER_ALLOCATOR at
// SUPACachingAllocator.cpp:3556, malloc :959, free :1224, round_size :1808),
// SUPAGuardImpl (C10_REGISTER_GUARD_IMPL at impl/SUPAGuardImpl.cpp:254),
// SUPAHooks, and the CPU fallback of aten/VariableFallbackKernel.cpp:31-64.
//
// Streams.  Each device has a default stream and a pool of 32 streams, all
// created non-blocking (so they never serialise with the legacy NULL stream
// other HIP code in the process uses) at the default priority; the current
// stream is thread-local per device, as SUPAStream.cpp:26-27,147 keeps it.
// A c10::Stream id is 0 for the default stream and 1..32 for the pool.
//
// Allocator design.  Device memory comes from hipMalloc in size classes
// (512 B granules below 1 MiB, 2 MiB granules above) and is cached per device
// and per stream on free: a block belongs to the stream current when it was
// allocated, and a freed block is reused only by allocations on that stream,
// which stream order makes safe.  record_stream(t, s) marks a block as used
// on another stream too; freeing it then records an event on each such
// stream and the block returns to its pool once every event has completed
// (the semantics of SUPACachingAllocator's recordStream, RecordStream.cpp:10-16).
// When hipMalloc fails the cache, including blocks still waiting on events
// (after waiting for them), is released and the allocation retried once
// before an OutOfMemoryError.  Blocks are never split, so a cached block is
// reused only by a request of at least half its size.
// PYTORCH_NO_SUPA_MEMORY_CACHING turns caching off (each free waits for the
// block's streams and calls hipFree), for device memory debugging.
#include <ATen/detail/PrivateUse1HooksInterface.h>
#include <ATen/native/CPUFallback.h>
#include <c10/core/Allocator.h>
#include <c10/core/impl/DeviceGuardImplInterface.h>
#include <c10/util/Exception.h>
#include <torch/library.h>

#include "generator.h"

#include <algorithm>
#include <atomic>
#include <cstdlib>
#include <cstring>
#include <sstream>
#include <map>
#include <mutex>
#include <unordered_map>
#include <vector>

#include "common.h"

namespace supa {

namespace {
bool env_on(const char* name) {
  const char* e = std::getenv(name);
  return e && *e && std::string(e) != "0";
}
// SUPA_LAUNCH_BLOCKING=1 or CUDA_LAUNCH_BLOCKING=1, the switches the
// reference reads (SUPAMiscFunctions.cpp:10-12): every launch is followed by
// a synchronisation of the current stream, so a kernel error (or an nll
// target out of range) is reported by the op that caused it.
const bool g_launch_blocking = env_on("SUPA_LAUNCH_BLOCKING") || env_on("CUDA_LAUNCH_BLOCKING");
}  // namespace

bool launch_blocking() { return g_launch_blocking; }

void check_status(int status, const char* what) {
  TORCH_CHECK(status == SUPA_AMD_OK, what, ": ", supa_amd_status_string(status), " (status ", status, ")",
              status > 0 && !g_launch_blocking
                  ? "\nsupa kernel errors can surface at a later call; SUPA_LAUNCH_BLOCKING=1 reports them at "
                    "the launch"
                  : "");
  if (g_launch_blocking) {
    const c10::DeviceIndex d = current_device();
    const hipError_t e = hipStreamSynchronize(current_stream(d));
    if (e != hipSuccess) (void)hipGetLastError();
    TORCH_CHECK(e == hipSuccess, what, ": kernel failed: ", hipGetErrorString(e));
    check_device_errors(d);
  }
}

bool dtype_supported(c10::ScalarType t) {
  switch (t) {
    case at::kByte: case at::kChar: case at::kShort: case at::kInt: case at::kLong:
    case at::kHalf: case at::kFloat: case at::kDouble: case at::kBool: case at::kBFloat16:
      return true;
    default:
      return false;
  }
}

// --------------------------------------------------------------- devices
namespace {
thread_local int tls_device = -1;

int query_device_count() {
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess) {
    (void)hipGetLastError();
    return 0;
  }
  return n;
}
}  // namespace

c10::DeviceIndex device_count() noexcept {
  static const int n = query_device_count();
  return static_cast<c10::DeviceIndex>(n);
}

c10::DeviceIndex current_device() {
  if (tls_device < 0) {
    int d = 0;
    SUPA_HIP_CHECK(hipGetDevice(&d));
    tls_device = d;
  }
  return static_cast<c10::DeviceIndex>(tls_device);
}

void set_device(c10::DeviceIndex d) {
  TORCH_CHECK(d >= 0 && d < device_count(), "supa: invalid device index ", int(d), " (", int(device_count()),
              " devices)");
  if (tls_device != d) {
    SUPA_HIP_CHECK(hipSetDevice(d));
    tls_device = d;
  }
}

// --------------------------------------------------------------- streams
namespace {
constexpr int kStreamDevices = 64;
constexpr int kPoolStreams = 32;

struct DeviceStreams {
  std::once_flag once;
  hipStream_t def = nullptr;
  hipStream_t pool[kPoolStreams] = {};
  std::atomic<uint32_t> next{0};
};
DeviceStreams g_streams[kStreamDevices];
thread_local c10::StreamId tls_stream[kStreamDevices] = {};

DeviceStreams& streams_of(c10::DeviceIndex d) {
  TORCH_CHECK(d >= 0 && d < kStreamDevices && d < device_count(), "supa: invalid device index ", int(d));
  DeviceStreams& ds = g_streams[d];
  std::call_once(ds.once, [&ds, d] {
    int prev = 0;
    SUPA_HIP_CHECK(hipGetDevice(&prev));
    SUPA_HIP_CHECK(hipSetDevice(d));
    SUPA_HIP_CHECK(hipStreamCreateWithFlags(&ds.def, hipStreamNonBlocking));
    for (auto& st : ds.pool) SUPA_HIP_CHECK(hipStreamCreateWithFlags(&st, hipStreamNonBlocking));
    SUPA_HIP_CHECK(hipSetDevice(prev));
  });
  return ds;
}
}  // namespace

hipStream_t stream_handle(c10::DeviceIndex d, c10::StreamId id) {
  DeviceStreams& ds = streams_of(d);
  if (id == 0) return ds.def;
  TORCH_CHECK(id >= 1 && id <= kPoolStreams, "supa: unknown stream id ", id, " on device ", int(d));
  return ds.pool[id - 1];
}

c10::Stream current_stream_obj(c10::DeviceIndex d) {
  (void)streams_of(d);
  return c10::Stream(c10::Stream::UNSAFE, c10::Device(kSupa, d), tls_stream[d]);
}

c10::Stream pool_stream(c10::DeviceIndex d) {
  DeviceStreams& ds = streams_of(d);
  const uint32_t k = ds.next.fetch_add(1) % kPoolStreams;
  return c10::Stream(c10::Stream::UNSAFE, c10::Device(kSupa, d), (c10::StreamId)(k + 1));
}

c10::Stream default_stream_obj(c10::DeviceIndex d) {
  (void)streams_of(d);
  return c10::Stream(c10::Stream::UNSAFE, c10::Device(kSupa, d), 0);
}

c10::Stream exchange_stream(const c10::Stream& s) {
  const c10::DeviceIndex d = s.device_index();
  (void)stream_handle(d, s.id());  // validates
  const c10::Stream old = current_stream_obj(d);
  tls_stream[d] = s.id();
  return old;
}

hipStream_t current_stream(c10::DeviceIndex d) {
  DeviceStreams& ds = streams_of(d);
  const c10::StreamId id = tls_stream[d];
  return id == 0 ? ds.def : ds.pool[id - 1];
}

void memcpy_h2d(void* dst, const void* src, size_t n, c10::DeviceIndex d) {
  const hipStream_t st = current_stream(d);
  SUPA_HIP_CHECK(hipMemcpyAsync(dst, src, n, hipMemcpyHostToDevice, st));
  SUPA_HIP_CHECK(hipStreamSynchronize(st));
}
void memcpy_d2h(void* dst, const void* src, size_t n, c10::DeviceIndex d) {
  const hipStream_t st = current_stream(d);
  SUPA_HIP_CHECK(hipMemcpyAsync(dst, src, n, hipMemcpyDeviceToHost, st));
  SUPA_HIP_CHECK(hipStreamSynchronize(st));
}

namespace {
constexpr int kScratchDevices = 64;
constexpr int kFlagSlots = 64;  // int32 slots in the 256-byte flag block: ids 0..kPoolStreams
static_assert(kPoolStreams + 1 <= kFlagSlots, "one error flag per stream");
std::mutex g_scratch_mu;
DeviceScratch g_scratch[kScratchDevices];

// Reads and clears flags [first, first + n) of device d on its current
// stream (which the caller has synchronised, or every stream has been), and
// raises the first error found.
void check_flags(c10::DeviceIndex d, int first, int n) {
  int32_t* flags = nullptr;
  {
    std::lock_guard<std::mutex> g(g_scratch_mu);
    if (d < 0 || d >= kScratchDevices || !g_scratch[d].error_flags) return;
    flags = g_scratch[d].error_flags;
  }
  int32_t h[kFlagSlots] = {};
  memcpy_d2h(h, flags + first, sizeof(int32_t) * n, d);
  int32_t code = 0;
  for (int i = 0; i < n; ++i) {
    if (h[i] != 0) {
      if (code == 0) code = h[i];
      const int32_t zero = 0;
      memcpy_h2d(flags + first + i, &zero, sizeof(zero), d);
    }
  }
  if (code != 0) {
    TORCH_CHECK_INDEX(code != 2, "supa: a kernel reported an out-of-bounds index (a scatter_ index outside the "
                                 "destination's size along dim)");
    TORCH_CHECK_INDEX(false, "supa: a kernel reported an out-of-bounds target index (nll_loss target outside "
                             "[0, n_classes) and not ignore_index)");
  }
}
}  // namespace

void synchronize(c10::DeviceIndex d) {
  const auto prev = current_device();
  set_device(d);
  SUPA_HIP_CHECK(hipDeviceSynchronize());
  set_device(prev);
  check_flags(d, 0, kPoolStreams + 1);  // every stream has drained
}

const DeviceScratch& device_scratch(c10::DeviceIndex d) {
  TORCH_CHECK(d >= 0 && d < kScratchDevices, "supa: device index out of range");
  std::lock_guard<std::mutex> g(g_scratch_mu);
  DeviceScratch& s = g_scratch[d];
  if (!s.error_flags) {
    const auto prev = current_device();
    if (prev != d) set_device(d);
    void* p = nullptr;
    SUPA_HIP_CHECK(hipMalloc(&p, sizeof(int32_t) * kFlagSlots));
    const hipStream_t st = stream_handle(d, 0);
    SUPA_HIP_CHECK(hipMemsetAsync(p, 0, sizeof(int32_t) * kFlagSlots, st));
    SUPA_HIP_CHECK(hipStreamSynchronize(st));
    s.error_flags = static_cast<int32_t*>(p);
    if (prev != d) set_device(prev);
  }
  return s;
}

int32_t* stream_error_flag(c10::DeviceIndex d) {
  int32_t* base = device_scratch(d).error_flags;
  (void)streams_of(d);
  return base + tls_stream[d];
}

void check_device_errors(c10::DeviceIndex d) {
  if (d < 0 || d >= kStreamDevices) return;
  check_flags(d, (int)tls_stream[d], 1);
}

// ------------------------------------------------------------- allocator
namespace {

constexpr int kMaxDevices = 64;

size_t round_size(size_t n) {
  if (n == 0) return 0;
  constexpr size_t kSmall = 512, kLarge = size_t(2) << 20, kSmallLimit = size_t(1) << 20;
  if (n < kSmallLimit) return (n + kSmall - 1) / kSmall * kSmall;
  return (n + kLarge - 1) / kLarge * kLarge;
}

struct Block {
  void* ptr;
  size_t size;
  int device;
  hipStream_t stream;                // the stream current at allocation: owns the block's reuse
  std::vector<hipStream_t> uses;     // other streams recorded by record_stream
};

// A freed block waiting for the events recorded on the streams that used it.
struct Pending {
  Block block;
  std::vector<hipEvent_t> events;
};

// upstream's format_size (the reference's OOM message uses it): bytes up to
// 1 KiB, then KiB / MiB / GiB with two decimals.
std::string format_size(uint64_t size) {
  std::ostringstream os;
  os.precision(2);
  os << std::fixed;
  if (size <= 1024) os << size << " bytes";
  else if (size <= 1048576) os << (double)size / 1024.0 << " KiB";
  else if (size <= 1073741824ULL) os << (double)size / 1048576.0 << " MiB";
  else os << (double)size / 1073741824.0 << " GiB";
  return os.str();
}

class CachingAllocator final : public c10::Allocator {
 public:
  c10::DataPtr allocate(size_t nbytes) override {
    const int dev = current_device();
    void* p = allocate_on(dev, current_stream(dev), nbytes);
    return {p, p, &CachingAllocator::raw_delete, c10::Device(kSupa, dev)};
  }

  // A block of nbytes for stream st of device dev (the current device);
  // nullptr for 0 bytes.  The reference refuses 1 EiB and more before
  // anything else (SUPACachingAllocator.cpp:3261-3263).
  void* allocate_on(int dev, hipStream_t st, size_t nbytes) {
    constexpr size_t kOneExaByte = size_t(1) << 60;
    TORCH_CHECK_WITH(OutOfMemoryError, nbytes < kOneExaByte,
                     "SUPA out of memory. Tried to allocate more than 1EB memory.");
    if (nbytes == 0) return nullptr;
    const size_t sz = round_size(nbytes);
    void* p = nullptr;
    if (!uncached_) {
      std::lock_guard<std::mutex> g(mu_);
      process_pending_locked(dev, false);
      p = take_cached_locked(dev, st, sz);
    }
    if (!p) p = device_malloc(dev, st, sz);
    return p;
  }

  // set_per_process_memory_fraction: the allocator reserves at most
  // fraction x the device's total memory; a request beyond it releases the
  // cache and then fails as out of memory.
  void set_fraction(int dev, double fraction) {
    size_t free_b = 0, total_b = 0;
    SUPA_HIP_CHECK(hipMemGetInfo(&free_b, &total_b));
    std::lock_guard<std::mutex> g(mu_);
    fraction_[dev] = fraction;
    limit_[dev] = (size_t)(fraction * (double)total_b);
  }
  double get_fraction(int dev) {
    std::lock_guard<std::mutex> g(mu_);
    return fraction_[dev];
  }

  c10::DeleterFnPtr raw_deleter() const override { return &CachingAllocator::raw_delete; }

  void copy_data(void* dest, const void* src, std::size_t count) const override {
    const int dev = current_device();
    const hipStream_t st = current_stream(dev);
    SUPA_HIP_CHECK(hipMemcpyAsync(dest, src, count, hipMemcpyDeviceToDevice, st));
    SUPA_HIP_CHECK(hipStreamSynchronize(st));
  }

  static void raw_delete(void* p) {
    if (p) instance().release(p);
  }

  static CachingAllocator& instance();

  // The block holding p is also used on stream st (record_stream): its reuse
  // waits for the work st has queued when the block is freed.
  void record_stream(void* p, hipStream_t st) {
    std::lock_guard<std::mutex> g(mu_);
    auto it = live_.find(p);
    TORCH_CHECK(it != live_.end(), "supa record_stream: pointer was not allocated by the supa caching allocator");
    Block& b = it->second;
    if (st == b.stream) return;
    if (std::find(b.uses.begin(), b.uses.end(), st) == b.uses.end()) b.uses.push_back(st);
  }

  void release(void* p) {
    std::lock_guard<std::mutex> g(mu_);
    auto it = live_.find(p);
    if (it == live_.end()) return;
    Block b = std::move(it->second);
    live_.erase(it);
    stats_[b.device].allocated -= (int64_t)b.size;
    stats_[b.device].num_frees += 1;
    if (uncached_) {
      // no caching: wait for every stream that used the block, then free it
      const int prev = current_device();
      if (prev != b.device) (void)hipSetDevice(b.device);
      (void)hipStreamSynchronize(b.stream);
      for (hipStream_t use : b.uses) (void)hipStreamSynchronize(use);
      (void)hipFree(b.ptr);
      (void)hipGetLastError();
      if (prev != b.device) (void)hipSetDevice(prev);
      stats_[b.device].reserved -= (int64_t)b.size;
      return;
    }
    if (b.uses.empty()) {
      free_[b.device][b.stream].emplace(b.size, b.ptr);
      return;
    }
    // an event on every other stream that used the block; reuse waits for all
    Pending pend;
    const int prev = current_device();
    if (prev != b.device) (void)hipSetDevice(b.device);
    for (hipStream_t use : b.uses) {
      hipEvent_t e = get_event_locked(b.device);
      const hipError_t rc = hipEventRecord(e, use);
      if (rc != hipSuccess) {
        (void)hipGetLastError();
        (void)hipStreamSynchronize(use);  // a stream that cannot take an event: wait for it instead
        events_[b.device].push_back(e);
        continue;
      }
      pend.events.push_back(e);
    }
    if (prev != b.device) (void)hipSetDevice(prev);
    b.uses.clear();
    pend.block = std::move(b);
    pending_[pend.block.device].push_back(std::move(pend));
  }

  void empty_cache() {
    std::lock_guard<std::mutex> g(mu_);
    for (int d = 0; d < kMaxDevices; ++d) process_pending_locked(d, true);
    release_cached_locked(-1);
  }

  AllocatorStats stats(int dev) {
    std::lock_guard<std::mutex> g(mu_);
    AllocatorStats s = stats_[dev];
    s.pending_blocks = (int64_t)pending_[dev].size();
    return s;
  }
  void reset_peak(int dev) {
    std::lock_guard<std::mutex> g(mu_);
    stats_[dev].peak_allocated = stats_[dev].allocated;
    stats_[dev].peak_reserved = stats_[dev].reserved;
  }
  // Test hook: the next `n` device allocations fail as if hipMalloc returned
  // hipErrorOutOfMemory (before and after the cache is released).
  void inject_oom(int n) {
    std::lock_guard<std::mutex> g(mu_);
    inject_oom_ = n;
  }

 private:
  void* take_cached_locked(int dev, hipStream_t st, size_t sz) {
    auto pit = free_[dev].find(st);
    if (pit == free_[dev].end()) return nullptr;
    auto& fl = pit->second;
    auto it = fl.lower_bound(sz);
    if (it == fl.end() || it->first > 2 * sz) return nullptr;
    void* p = it->second;
    const size_t bsz = it->first;
    fl.erase(it);
    live_[p] = Block{p, bsz, dev, st, {}};
    account_alloc(dev, bsz, false);
    return p;
  }

  hipEvent_t get_event_locked(int dev) {
    auto& pool = events_[dev];
    if (!pool.empty()) {
      hipEvent_t e = pool.back();
      pool.pop_back();
      return e;
    }
    hipEvent_t e;
    SUPA_HIP_CHECK(hipEventCreateWithFlags(&e, hipEventDisableTiming));
    return e;
  }

  // Moves freed blocks whose events have all completed to their stream's
  // pool; with wait, waits for every event first.
  void process_pending_locked(int dev, bool wait) {
    auto& pl = pending_[dev];
    for (size_t i = 0; i < pl.size();) {
      bool done = true;
      for (hipEvent_t e : pl[i].events) {
        const hipError_t rc = wait ? hipEventSynchronize(e) : hipEventQuery(e);
        if (rc == hipErrorNotReady) {
          (void)hipGetLastError();
          done = false;
          break;
        }
        if (rc != hipSuccess) (void)hipGetLastError();
      }
      if (!done) {
        ++i;
        continue;
      }
      for (hipEvent_t e : pl[i].events) events_[dev].push_back(e);
      const Block& b = pl[i].block;
      free_[dev][b.stream].emplace(b.size, b.ptr);
      pl[i] = std::move(pl.back());
      pl.pop_back();
    }
  }

  void account_alloc(int dev, size_t bsz, bool fresh) {
    auto& s = stats_[dev];
    s.allocated += (int64_t)bsz;
    s.peak_allocated = std::max(s.peak_allocated, s.allocated);
    s.num_allocs += 1;
    if (fresh) {
      s.reserved += (int64_t)bsz;
      s.peak_reserved = std::max(s.peak_reserved, s.reserved);
      s.num_device_mallocs += 1;
    }
  }

  void release_cached_locked(int dev) {
    const int prev = current_device();
    for (int d = 0; d < kMaxDevices; ++d) {
      if (dev >= 0 && d != dev) continue;
      if (free_[d].empty()) continue;
      (void)hipSetDevice(d);
      for (auto& pool : free_[d]) {
        for (auto& kv : pool.second) {
          (void)hipFree(kv.second);
          stats_[d].reserved -= (int64_t)kv.first;
        }
      }
      free_[d].clear();
    }
    (void)hipSetDevice(prev);
  }

  // hipMalloc, unless a test hook fails it, the request cannot fit the
  // device at all (no driver call for it), or it would take the reserved
  // bytes past the memory-fraction limit.
  hipError_t try_malloc(int dev, void** p, size_t sz, size_t total) {
    {
      std::lock_guard<std::mutex> g(mu_);
      if (inject_oom_ > 0) {
        --inject_oom_;
        return hipErrorOutOfMemory;
      }
      if (sz > total) return hipErrorOutOfMemory;
      if (limit_[dev] != SIZE_MAX && (size_t)stats_[dev].reserved + sz > limit_[dev]) return hipErrorOutOfMemory;
    }
    return hipMalloc(p, sz);
  }

  void* device_malloc(int dev, hipStream_t st, size_t sz) {
    void* p = nullptr;
    size_t free_b = 0, total_b = 0;
    if (hipMemGetInfo(&free_b, &total_b) != hipSuccess) {
      (void)hipGetLastError();
      total_b = SIZE_MAX;
    }
    hipError_t e = try_malloc(dev, &p, sz, total_b);
    if (e != hipSuccess) {
      (void)hipGetLastError();
      {
        std::lock_guard<std::mutex> g(mu_);
        process_pending_locked(dev, true);
        release_cached_locked(dev);
        stats_[dev].num_ooms_retried += 1;
      }
      e = try_malloc(dev, &p, sz, total_b);
    }
    if (e != hipSuccess) {
      (void)hipGetLastError();
      (void)hipMemGetInfo(&free_b, &total_b);
      (void)hipGetLastError();
      AllocatorStats s = stats(dev);
      std::string allowed;
      {
        std::lock_guard<std::mutex> g(mu_);
        if (limit_[dev] != SIZE_MAX) allowed = format_size(limit_[dev]) + " allowed; ";
      }
      // the reference's message (SUPACachingAllocator.cpp:1080-1101), so that
      // code matching on it keeps working
      TORCH_CHECK_WITH(OutOfMemoryError, false, "SUPA out of memory. Tried to allocate ", format_size(sz), ". GPU ",
                       dev, " has a total capacity of ", format_size(total_b), " of which ", format_size(free_b),
                       " is free. ", allowed, "Of the allocated memory ", format_size(s.allocated),
                       " is allocated by PyTorch, and ", format_size(s.reserved - s.allocated),
                       " is reserved by PyTorch but unallocated.");
    }
    std::lock_guard<std::mutex> g(mu_);
    live_[p] = Block{p, sz, dev, st, {}};
    account_alloc(dev, sz, true);
    return p;
  }

  // PYTORCH_NO_SUPA_MEMORY_CACHING (any value), as the reference reads it
  // (SUPACachingAllocator.cpp:2975-2978): every block goes to hipMalloc and
  // back to hipFree, so device memory checkers see each allocation.
  const bool uncached_ = std::getenv("PYTORCH_NO_SUPA_MEMORY_CACHING") != nullptr;
  std::mutex mu_;
  std::map<hipStream_t, std::multimap<size_t, void*>> free_[kMaxDevices];
  std::vector<Pending> pending_[kMaxDevices];
  std::vector<hipEvent_t> events_[kMaxDevices];
  std::unordered_map<void*, Block> live_;
  AllocatorStats stats_[kMaxDevices];
  double fraction_[kMaxDevices] = {};
  size_t limit_[kMaxDevices] = {};
  int inject_oom_ = 0;

 public:
  CachingAllocator() {
    for (int d = 0; d < kMaxDevices; ++d) {
      fraction_[d] = 1.0;
      limit_[d] = SIZE_MAX;
    }
  }
};

// Pinned host memory (pin_memory(), pin_memory=True, the accelerator's host
// allocator): hipHostMalloc blocks in power-of-two size classes from 4 KiB,
// cached on free and returned to the driver only by empty_host_cache.  Copies
// between the host and a supa device are synchronous in this build, so a
// freed block can be reused at once.
class PinnedAllocator final : public c10::Allocator {
 public:
  c10::DataPtr allocate(size_t nbytes) override {
    if (nbytes == 0) return {nullptr, nullptr, &PinnedAllocator::raw_delete, c10::Device(c10::DeviceType::CPU)};
    size_t sz = 4096;
    while (sz < nbytes) sz <<= 1;
    void* p = nullptr;
    {
      std::lock_guard<std::mutex> g(mu_);
      auto it = free_.find(sz);
      if (it != free_.end()) {
        p = it->second;
        free_.erase(it);
      }
    }
    if (!p) {
      hipError_t e = hipHostMalloc(&p, sz, hipHostMallocDefault);
      if (e != hipSuccess) {
        (void)hipGetLastError();
        empty_cache();
        e = hipHostMalloc(&p, sz, hipHostMallocDefault);
      }
      if (e != hipSuccess) {
        (void)hipGetLastError();
        TORCH_CHECK_WITH(OutOfMemoryError, false, "SUPA out of memory. Tried to allocate ", format_size(sz),
                         " of pinned host memory.");
      }
    }
    std::lock_guard<std::mutex> g(mu_);
    live_[p] = sz;
    return {p, p, &PinnedAllocator::raw_delete, c10::Device(c10::DeviceType::CPU)};
  }
  c10::DeleterFnPtr raw_deleter() const override { return &PinnedAllocator::raw_delete; }
  void copy_data(void* dest, const void* src, std::size_t count) const override { std::memcpy(dest, src, count); }

  static void raw_delete(void* p) {
    if (!p) return;
    PinnedAllocator& a = instance();
    std::lock_guard<std::mutex> g(a.mu_);
    auto it = a.live_.find(p);
    if (it == a.live_.end()) return;
    a.free_.emplace(it->second, p);
    a.live_.erase(it);
  }
  void empty_cache() {
    std::lock_guard<std::mutex> g(mu_);
    for (auto& kv : free_) (void)hipHostFree(kv.second);
    (void)hipGetLastError();
    free_.clear();
  }
  static PinnedAllocator& instance() {
    static PinnedAllocator* a = new PinnedAllocator();  // never destroyed: frees can arrive at exit
    return *a;
  }

 private:
  std::mutex mu_;
  std::multimap<size_t, void*> free_;
  std::unordered_map<void*, size_t> live_;
};

CachingAllocator& CachingAllocator::instance() {
  static CachingAllocator* a = new CachingAllocator();  // never destroyed: frees can arrive at exit
  return *a;
}

struct AllocatorRegistrar {
  AllocatorRegistrar() { c10::SetAllocator(kSupa, &CachingAllocator::instance()); }
};
AllocatorRegistrar g_allocator_registrar;

}  // namespace

c10::Allocator* allocator() { return &CachingAllocator::instance(); }
AllocatorStats allocator_stats(c10::DeviceIndex d) { return CachingAllocator::instance().stats(d); }
void allocator_record_stream(void* ptr, const c10::Stream& s) {
  CachingAllocator::instance().record_stream(ptr, stream_handle(s.device_index(), s.id()));
}
void allocator_inject_oom(int n) { CachingAllocator::instance().inject_oom(n); }
void allocator_reset_peak(c10::DeviceIndex d) { CachingAllocator::instance().reset_peak(d); }
void allocator_empty_cache() { CachingAllocator::instance().empty_cache(); }
void pinned_empty_cache() { PinnedAllocator::instance().empty_cache(); }
void* allocator_raw_alloc(size_t nbytes, c10::DeviceIndex d, hipStream_t st) {
  const auto prev = current_device();
  if (d != prev) set_device(d);
  void* p = CachingAllocator::instance().allocate_on(d, st, nbytes);
  if (d != prev) set_device(prev);
  return p;
}
void allocator_raw_delete(void* p) { CachingAllocator::raw_delete(p); }
void allocator_set_memory_fraction(double fraction, c10::DeviceIndex d) {
  const auto prev = current_device();
  if (d != prev) set_device(d);
  CachingAllocator::instance().set_fraction(d, fraction);
  if (d != prev) set_device(prev);
}
double allocator_get_memory_fraction(c10::DeviceIndex d) { return CachingAllocator::instance().get_fraction(d); }

at::Tensor empty_strided_supa(c10::IntArrayRef size, c10::IntArrayRef stride, c10::ScalarType dtype,
                              c10::DeviceIndex device) {
  const auto prev = current_device();
  if (device >= 0 && device != prev) set_device(device);
  const c10::DispatchKeySet ks(c10::DispatchKey::PrivateUse1);
  at::Tensor t = at::detail::empty_strided_generic(size, stride, allocator(), ks, dtype);
  if (device >= 0 && device != prev) set_device(prev);
  return t;
}

at::Tensor empty_supa(c10::IntArrayRef size, c10::ScalarType dtype, c10::DeviceIndex device,
                      c10::MemoryFormat fmt) {
  const auto prev = current_device();
  if (device >= 0 && device != prev) set_device(device);
  const c10::DispatchKeySet ks(c10::DispatchKey::PrivateUse1);
  at::Tensor t = at::detail::empty_generic(size, allocator(), ks, dtype, fmt);
  if (device >= 0 && device != prev) set_device(prev);
  return t;
}

// ------------------------------------------------------------ guard impl
namespace {

struct SupaGuardImpl final : public c10::impl::DeviceGuardImplInterface {
  c10::DeviceType type() const override { return kSupa; }
  c10::Device exchangeDevice(c10::Device d) const override {
    const auto old = current_device();
    if (d.index() != old) set_device(d.index());
    return c10::Device(kSupa, old);
  }
  c10::Device getDevice() const override { return c10::Device(kSupa, current_device()); }
  void setDevice(c10::Device d) const override { set_device(d.index()); }
  void uncheckedSetDevice(c10::Device d) const noexcept override {
    if (hipSetDevice(d.index()) == hipSuccess) tls_device = d.index();
  }
  // a device without an index (torch.Stream("supa")) is the current device
  static c10::DeviceIndex index_of(c10::Device d) { return d.has_index() ? d.index() : current_device(); }
  c10::Stream getStream(c10::Device d) const override { return current_stream_obj(index_of(d)); }
  c10::Stream getDefaultStream(c10::Device d) const override { return default_stream_obj(index_of(d)); }
  c10::Stream getStreamFromGlobalPool(c10::Device d, bool /*high_priority*/) const override {
    return pool_stream(index_of(d));  // every stream has the default priority
  }
  c10::Stream getNewStream(c10::Device d, int /*priority*/) const override { return pool_stream(index_of(d)); }
  c10::Stream exchangeStream(c10::Stream s) const override { return exchange_stream(s); }
  c10::DeviceIndex deviceCount() const noexcept override { return device_count(); }

  void destroyEvent(void* event, const c10::DeviceIndex /*device_index*/) const noexcept override {
    if (event) (void)hipEventDestroy(static_cast<hipEvent_t>(event));
  }
  void record(void** event, const c10::Stream& stream, const c10::DeviceIndex device_index,
              const c10::EventFlag flag) const override {
    TORCH_CHECK(device_index == -1 || device_index == stream.device_index(), "supa event and stream devices differ");
    const auto prev = current_device();
    if (stream.device_index() != prev) set_device(stream.device_index());
    if (!*event) {
      hipEvent_t e;
      // as the CUDA guard: PYTORCH_DEFAULT events skip timing, BACKEND_DEFAULT
      // ones (torch.Event(enable_timing=True)) keep it
      SUPA_HIP_CHECK(hipEventCreateWithFlags(
          &e, flag == c10::EventFlag::PYTORCH_DEFAULT ? hipEventDisableTiming : hipEventDefault));
      *event = e;
    }
    SUPA_HIP_CHECK(hipEventRecord(static_cast<hipEvent_t>(*event), stream_handle(stream.device_index(), stream.id())));
    if (stream.device_index() != prev) set_device(prev);
  }
  void block(void* event, const c10::Stream& stream) const override {
    if (!event) return;
    SUPA_HIP_CHECK(hipStreamWaitEvent(stream_handle(stream.device_index(), stream.id()),
                                      static_cast<hipEvent_t>(event), 0));
  }
  bool queryEvent(void* event) const override {
    if (!event) return true;
    const hipError_t e = hipEventQuery(static_cast<hipEvent_t>(event));
    if (e == hipErrorNotReady) {
      (void)hipGetLastError();
      return false;
    }
    SUPA_HIP_CHECK(e);
    return true;
  }
  bool queryStream(const c10::Stream& stream) const override {
    const hipError_t e = hipStreamQuery(stream_handle(stream.device_index(), stream.id()));
    if (e == hipErrorNotReady) {
      (void)hipGetLastError();
      return false;
    }
    SUPA_HIP_CHECK(e);
    return true;
  }
  void synchronizeStream(const c10::Stream& stream) const override {
    SUPA_HIP_CHECK(hipStreamSynchronize(stream_handle(stream.device_index(), stream.id())));
  }
  void synchronizeEvent(void* event) const override {
    if (event) SUPA_HIP_CHECK(hipEventSynchronize(static_cast<hipEvent_t>(event)));
  }
  void synchronizeDevice(const c10::DeviceIndex device_index) const override { synchronize(device_index); }
  void recordDataPtrOnStream(const c10::DataPtr& data_ptr, const c10::Stream& stream) const override {
    if (data_ptr.get()) allocator_record_stream(data_ptr.get(), stream);
  }
  double elapsedTime(void* e1, void* e2, const c10::DeviceIndex /*device_index*/) const override {
    float ms = 0.f;
    SUPA_HIP_CHECK(hipEventElapsedTime(&ms, static_cast<hipEvent_t>(e1), static_cast<hipEvent_t>(e2)));
    return ms;
  }
};

C10_REGISTER_GUARD_IMPL(PrivateUse1, SupaGuardImpl);

// ------------------------------------------------------------------ hooks
struct SupaHooks final : public at::PrivateUse1HooksInterface {
  bool isBuilt() const override { return true; }
  bool isAvailable() const override { return device_count() > 0; }
  bool hasPrimaryContext(c10::DeviceIndex device_index) const override {
    return device_index >= 0 && device_index < device_count();
  }
  c10::DeviceIndex deviceCount() const override { return device_count(); }
  void setCurrentDevice(c10::DeviceIndex device) const override { set_device(device); }
  c10::DeviceIndex getCurrentDevice() const override { return current_device(); }
  c10::DeviceIndex exchangeDevice(c10::DeviceIndex device) const override {
    const auto old = current_device();
    set_device(device);
    return old;
  }
  c10::DeviceIndex maybeExchangeDevice(c10::DeviceIndex device) const override { return exchangeDevice(device); }
  at::Device getDeviceFromPtr(void* data) const override {
    hipPointerAttribute_t attr;
    if (hipPointerGetAttributes(&attr, data) == hipSuccess) return at::Device(kSupa, attr.device);
    (void)hipGetLastError();
    return at::Device(kSupa, current_device());
  }
  const at::Generator& getDefaultGenerator(c10::DeviceIndex device_index) const override {
    return default_generator(device_index);
  }
  at::Generator getNewGenerator(c10::DeviceIndex device_index) const override { return new_generator(device_index); }
  // any address inside page-locked host memory (an interior pointer of a
  // pinned block too), as the HIP runtime reports it
  bool isPinnedPtr(const void* data) const override {
    if (!data) return false;
    hipPointerAttribute_t attr;
    if (hipPointerGetAttributes(&attr, data) != hipSuccess) {
      (void)hipGetLastError();
      return false;
    }
    return attr.type == hipMemoryTypeHost;
  }
  at::Allocator* getPinnedMemoryAllocator() const override { return &PinnedAllocator::instance(); }
  void resizePrivateUse1Bytes(const c10::Storage& storage, size_t newsize) const override {
    // grow or shrink by reallocating and copying the overlap
    c10::StorageImpl* impl = storage.unsafeGetStorageImpl();
    const size_t old = impl->nbytes();
    if (newsize == old) return;
    c10::DataPtr fresh = allocator()->allocate(newsize);
    const size_t n = std::min(old, newsize);
    if (n > 0)
      SUPA_HIP_CHECK(hipMemcpyAsync(fresh.get(), impl->data(), n, hipMemcpyDeviceToDevice,
                                    current_stream(current_device())));
    impl->set_data_ptr_noswap(std::move(fresh));
    impl->set_nbytes(newsize);
  }
};

struct HooksRegistrar {
  HooksRegistrar() { at::RegisterPrivateUse1HooksInterface(new SupaHooks()); }
};
HooksRegistrar g_hooks_registrar;

// --------------------------------------------------------- CPU fallback
std::atomic<bool> g_fallback_enabled{[] {
  const char* e = std::getenv("SUPA_AMD_CPU_FALLBACK");
  return !(e && std::string(e) == "0");
}()};
std::mutex g_fb_mu;
std::map<std::string, int64_t> g_fb_counts;

}  // namespace

void supa_cpu_fallback(const c10::OperatorHandle& op, torch::jit::Stack* stack) {
  const std::string name = c10::toString(op.schema().operator_name());
  {
    std::lock_guard<std::mutex> g(g_fb_mu);
    g_fb_counts[name] += 1;
  }
  TORCH_CHECK(g_fallback_enabled.load(), "supa: operator ", name,
              " has no supa kernel and the CPU fallback is disabled");
  at::native::cpu_fallback(op, stack);
}

void set_cpu_fallback_enabled(bool on) { g_fallback_enabled.store(on); }
bool cpu_fallback_enabled() { return g_fallback_enabled.load(); }

namespace {
// -1: the reference's routing (float32 fused, 16-bit decomposed); 0: none
// fused; 1: every floating dtype fused.  SUPA_AMD_FUSED_CE=0 / 1 sets the
// start value.
std::atomic<int> g_fused_ce{[] {
  const char* e = std::getenv("SUPA_AMD_FUSED_CE");
  if (e && std::string(e) == "1") return 1;
  if (e && std::string(e) == "0") return 0;
  return -1;
}()};
}  // namespace
void set_fused_cross_entropy_mode(int mode) { g_fused_ce.store(mode < 0 ? -1 : (mode > 0 ? 1 : 0)); }
int fused_cross_entropy_mode() { return g_fused_ce.load(); }

namespace {
std::atomic<bool> g_fused_bce{[] {
  const char* e = std::getenv("SUPA_AMD_FUSED_BCE");
  return !(e && std::string(e) == "0");
}()};
}  // namespace
void set_fused_bce_backward_enabled(bool on) { g_fused_bce.store(on); }
bool fused_bce_backward_enabled() { return g_fused_bce.load(); }

namespace {
std::atomic<bool> g_accurate_gelu{[] {
  const char* e = std::getenv("SUPA_AMD_ACCURATE_GELU");
  return e && std::string(e) == "1";
}()};
}  // namespace
void set_accurate_gelu_enabled(bool on) { g_accurate_gelu.store(on); }
bool accurate_gelu_enabled() { return g_accurate_gelu.load(); }
std::vector<std::pair<std::string, int64_t>> fallback_counts() {
  std::lock_guard<std::mutex> g(g_fb_mu);
  return {g_fb_counts.begin(), g_fb_counts.end()};
}
void reset_fallback_counts() {
  std::lock_guard<std::mutex> g(g_fb_mu);
  g_fb_counts.clear();
}

}  // namespace supa

TORCH_LIBRARY_IMPL(_, PrivateUse1, m) {
  m.fallback(torch::CppFunction::makeFromBoxedFunction<&supa::supa_cpu_fallback>());
}

namespace {
// Tensor.record_stream(s): the tensor's block is also used on stream s
// (replaces the reference's aten/ops/RecordStream.cpp:10-16).
void record_stream_supa(at::Tensor& self, c10::Stream s) {
  TORCH_CHECK(s.device_type() == supa::kSupa, "record_stream: expected a supa stream, got ", s);
  TORCH_CHECK(self.device() == s.device(), "record_stream: tensor on ", self.device(), ", stream on ", s.device());
  supa::allocator_record_stream(self.storage().data_ptr().get(), s);
}
}  // namespace

namespace {
// tensor.data = other across the host and the device: upstream counts only
// its own dense backends as shallow-copy compatible; a supa tensor and a CPU
// tensor are both dense storages here too (the reference's
// aten/ops/HasCompatibleShallowCopyType.cpp:12-23).  Registered for the supa
// keys, so dispatch reaches it whenever either tensor is on the device.
bool has_compatible_shallow_copy_type_supa(const at::Tensor& self, const at::Tensor& from) {
  const c10::DispatchKeySet a = self.key_set(), b = from.key_set();
  auto dense = [](c10::DispatchKeySet ks) {
    return ks.has(c10::DispatchKey::CPU) || ks.has(c10::DispatchKey::PrivateUse1);
  };
  return a == b || (dense(a) && dense(b));
}
}  // namespace

TORCH_LIBRARY_IMPL(aten, PrivateUse1, m) {
  m.impl("record_stream", TORCH_FN(record_stream_supa));
  m.impl("_has_compatible_shallow_copy_type", TORCH_FN(has_compatible_shallow_copy_type_supa));
}
TORCH_LIBRARY_IMPL(aten, AutogradPrivateUse1, m) {
  m.impl("_has_compatible_shallow_copy_type", TORCH_FN(has_compatible_shallow_copy_type_supa));
}

