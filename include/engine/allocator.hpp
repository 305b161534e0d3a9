#pragma once
//===----------------------------------------------------------------------===//
// engine/allocator.hpp -- allocator interface, statistics and the passthrough.
//
// Contract of the reference (include/engine/allocator.hpp:34-63,
// src/allocator.cpp:22-118): AllocStats with exact counters and a one-line
// to_string(); an Allocator interface whose allocate() returns memory aligned
// to at least 256 bytes; default_allocator(Device) forwards every request to
// the driver (host aligned_alloc / hipMalloc) and counts it. Backed by the
// C-ABI (eng_passthrough_*).
//===----------------------------------------------------------------------===//

#include <engine/tensor.hpp>

#include <cstddef>
#include <cstdio>
#include <string>

namespace engine {

struct AllocStats {
  std::size_t bytes_in_use = 0;
  std::size_t bytes_reserved = 0;
  std::size_t peak_bytes_in_use = 0;
  std::size_t num_allocs = 0;
  std::size_t num_driver_allocs = 0;  ///< the pool works iff this stays tiny

  std::string to_string() const {
    auto mib = [](std::size_t b) { return static_cast<double>(b) / (1024.0 * 1024.0); };
    char buf[256];
    std::snprintf(buf, sizeof(buf),
                  "in_use=%.2f MiB, reserved=%.2f MiB, peak=%.2f MiB, allocs=%zu, driver_allocs=%zu",
                  mib(bytes_in_use), mib(bytes_reserved), mib(peak_bytes_in_use), num_allocs,
                  num_driver_allocs);
    return buf;
  }
};

inline AllocStats to_alloc_stats(const eng_alloc_stats& s) {
  AllocStats out;
  out.bytes_in_use = static_cast<std::size_t>(s.bytes_in_use);
  out.bytes_reserved = static_cast<std::size_t>(s.bytes_reserved);
  out.peak_bytes_in_use = static_cast<std::size_t>(s.peak_bytes_in_use);
  out.num_allocs = static_cast<std::size_t>(s.num_allocs);
  out.num_driver_allocs = static_cast<std::size_t>(s.num_driver_allocs);
  return out;
}

class Allocator {
 public:
  virtual ~Allocator() = default;
  /// At least `bytes`, aligned to at least 256 bytes; nullptr for 0 bytes.
  virtual void* allocate(std::size_t bytes) = 0;
  virtual void deallocate(void* ptr) = 0;
  virtual Device device() const = 0;
  virtual AllocStats stats() const = 0;
};

namespace detail {
class PassthroughAllocator final : public Allocator {
 public:
  explicit PassthroughAllocator(Device d) : device_(d) {}
  void* allocate(std::size_t bytes) override {
    void* p = nullptr;
    ENGINE_ABI_CHECK(eng_passthrough_allocate(static_cast<int>(device_), bytes, &p));
    return p;
  }
  void deallocate(void* ptr) override {
    ENGINE_ABI_CHECK(eng_passthrough_deallocate(static_cast<int>(device_), ptr));
  }
  Device device() const override { return device_; }
  AllocStats stats() const override {
    eng_alloc_stats s{};
    ENGINE_ABI_CHECK(eng_passthrough_stats(static_cast<int>(device_), &s));
    return to_alloc_stats(s);
  }

 private:
  Device device_;
};
}  // namespace detail

/// Passthrough allocator of a device: correct, slow, the pool's baseline.
inline Allocator& default_allocator(Device device) {
  static detail::PassthroughAllocator cpu(Device::CPU);
  static detail::PassthroughAllocator gpu(Device::HIP);
  return device == Device::CPU ? static_cast<Allocator&>(cpu) : static_cast<Allocator&>(gpu);
}

}  // namespace engine
