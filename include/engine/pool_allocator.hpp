#pragma once
//===----------------------------------------------------------------------===//
// engine/pool_allocator.hpp -- pooled allocator with stream-ordered reuse.
//
// Contract of the reference (include/engine/pool_allocator.hpp:27-148,
// src/pool_allocator.cpp:38-271); the pool itself lives in libengine_hip.so
// behind eng_pool_* (power-of-two buckets >= 256 B, 256-B alignment, slabs
// doubling from the initial size up to 64 MiB, GPU blocks reused only after
// the stream they were freed on has passed the free point, exact stats).
//===----------------------------------------------------------------------===//

#include <engine/allocator.hpp>

#include <hip/hip_runtime_api.h>

#include <cstddef>

namespace engine {

class PoolAllocator final : public Allocator {
 public:
  explicit PoolAllocator(Device device, std::size_t initial_slab_size = 4 * 1024 * 1024)
      : device_(device), owned_(true) {
    ENGINE_ABI_CHECK(eng_pool_create(&pool_, static_cast<int>(device), initial_slab_size));
  }
  ~PoolAllocator() override {
    if (owned_ && pool_ != nullptr) (void)eng_pool_destroy(pool_);
  }

  PoolAllocator(const PoolAllocator&) = delete;
  PoolAllocator& operator=(const PoolAllocator&) = delete;

  void* allocate(std::size_t bytes) override {
    void* p = nullptr;
    ENGINE_ABI_CHECK(eng_pool_allocate(pool_, bytes, &p));
    return p;
  }

  /// Host pools: immediate. GPU pools: reuse deferred past the default stream's
  /// current work.
  void deallocate(void* ptr) override { deallocate(ptr, nullptr); }

  /// Returns `ptr` to the pool once all work queued on `stream` so far finishes.
  void deallocate(void* ptr, hipStream_t stream) {
    ENGINE_ABI_CHECK(eng_pool_deallocate(pool_, ptr, stream));
  }

  Device device() const override { return device_; }

  AllocStats stats() const override {
    eng_alloc_stats s{};
    ENGINE_ABI_CHECK(eng_pool_stats(pool_, &s));
    return to_alloc_stats(s);
  }

  /// Releases every slab and resets the statistics.
  void reset() { ENGINE_ABI_CHECK(eng_pool_reset(pool_)); }

  eng_pool handle() const { return pool_; }

  /// Wraps a library-owned pool (the process-wide ones) without owning it.
  static PoolAllocator& wrap_default(Device device) {
    static PoolAllocator cpu(Device::CPU, Borrow{});
    static PoolAllocator gpu(Device::HIP, Borrow{});
    return device == Device::CPU ? cpu : gpu;
  }

 private:
  struct Borrow {};
  PoolAllocator(Device device, Borrow) : device_(device), owned_(false) {
    ENGINE_ABI_CHECK(eng_pool_default(&pool_, static_cast<int>(device)));
  }

  Device device_;
  bool owned_;
  eng_pool pool_ = nullptr;
};

/// RAII scratch from a PoolAllocator; on GPU pools the release is bound to the
/// launch stream so another stream cannot reuse the block too early.
class ScopedPoolBuffer {
 public:
  ScopedPoolBuffer(PoolAllocator& pool, std::size_t bytes) : pool_(pool), ptr_(pool.allocate(bytes)) {}
  ScopedPoolBuffer(PoolAllocator& pool, std::size_t bytes, hipStream_t stream)
      : pool_(pool), ptr_(pool.allocate(bytes)), stream_(stream) {}
  ~ScopedPoolBuffer() {
    try {
      release();
    } catch (...) {
    }
  }

  ScopedPoolBuffer(const ScopedPoolBuffer&) = delete;
  ScopedPoolBuffer& operator=(const ScopedPoolBuffer&) = delete;
  ScopedPoolBuffer(ScopedPoolBuffer&&) = delete;
  ScopedPoolBuffer& operator=(ScopedPoolBuffer&&) = delete;

  void* get() const { return ptr_; }
  template <typename T>
  T* as() const {
    return static_cast<T*>(ptr_);
  }

  void release() {
    if (ptr_ == nullptr) return;
    void* p = ptr_;
    ptr_ = nullptr;
    pool_.deallocate(p, stream_);
  }

 private:
  PoolAllocator& pool_;
  void* ptr_ = nullptr;
  hipStream_t stream_ = nullptr;
};

/// The process-wide pool of a device (created on first use).
inline PoolAllocator& pool_allocator(Device device) { return PoolAllocator::wrap_default(device); }

}  // namespace engine
