#pragma once
//===----------------------------------------------------------------------===//
// engine/device_buffer.hpp -- owning, move-only device array.
//
// The reference's DeviceBuffer<T> contract (include/engine/device_buffer.hpp:
// 29-101): allocate `count` elements on the device, upload / download whole
// vectors (sizes must match), zero, get / size / bytes; move-only so a device
// copy is never hidden behind `=`; the destructor never throws. Memory comes
// from the C-ABI (eng_malloc / eng_memcpy_*), i.e. hipMalloc.
//===----------------------------------------------------------------------===//

#include <engine/check.hpp>

#include <cstddef>
#include <vector>

namespace engine {

template <typename T>
class DeviceBuffer {
 public:
  DeviceBuffer() = default;

  explicit DeviceBuffer(std::size_t count) : count_(count) {
    if (count_ > 0) {
      void* p = nullptr;
      ENGINE_ABI_CHECK(eng_malloc(&p, count_ * sizeof(T)));
      ptr_ = static_cast<T*>(p);
    }
  }

  explicit DeviceBuffer(const std::vector<T>& host) : DeviceBuffer(host.size()) { upload(host); }

  ~DeviceBuffer() {
    if (ptr_ != nullptr) (void)eng_free(ptr_);
  }

  DeviceBuffer(const DeviceBuffer&) = delete;
  DeviceBuffer& operator=(const DeviceBuffer&) = delete;

  DeviceBuffer(DeviceBuffer&& o) noexcept : ptr_(o.ptr_), count_(o.count_) {
    o.ptr_ = nullptr;
    o.count_ = 0;
  }

  DeviceBuffer& operator=(DeviceBuffer&& o) noexcept {
    if (this != &o) {
      if (ptr_ != nullptr) (void)eng_free(ptr_);
      ptr_ = o.ptr_;
      count_ = o.count_;
      o.ptr_ = nullptr;
      o.count_ = 0;
    }
    return *this;
  }

  void upload(const std::vector<T>& host) {
    ENGINE_CHECK(host.size() == count_, "upload(): host/device element count mismatch");
    if (count_ > 0) ENGINE_ABI_CHECK(eng_memcpy_h2d(ptr_, host.data(), bytes()));
  }

  std::vector<T> download() const {
    std::vector<T> host(count_);
    if (count_ > 0) ENGINE_ABI_CHECK(eng_memcpy_d2h(host.data(), ptr_, bytes()));
    return host;
  }

  void zero() {
    if (count_ > 0) ENGINE_ABI_CHECK(eng_memset(ptr_, 0, bytes()));
  }

  T* get() { return ptr_; }
  const T* get() const { return ptr_; }
  std::size_t size() const { return count_; }
  std::size_t bytes() const { return count_ * sizeof(T); }

 private:
  T* ptr_ = nullptr;
  std::size_t count_ = 0;
};

}  // namespace engine
