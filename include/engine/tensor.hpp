#pragma once
//===----------------------------------------------------------------------===//
// engine/tensor.hpp -- Storage (owning or borrowed bytes) and Tensor (views).
//
// Contract of the reference (include/engine/tensor.hpp:50-195,
// src/tensor.cpp:56-560), header-only here and HIP-backed:
//   * Storage owns `bytes` on one device (host malloc / eng_malloc) or borrows
//     an external pointer it never frees;
//   * Tensor is shape + strides (in elements) + element offset + dtype over a
//     shared Storage; reshape/permute/transpose/slice are metadata edits;
//     contiguous/clone/to copy;
//   * numel() of an undefined tensor is 0, of a 0-d tensor 1; an axis of size 0
//     makes the tensor empty (and contiguous by convention);
//   * reshape requires a contiguous tensor and allows one -1;
//   * contiguous() of a non-contiguous GPU tensor is an error (pack on host);
//   * ptr<T>(device) checks device and element size.
// Device numbering matches the C-ABI: CPU = 0, HIP = 1. `Device::CUDA` names
// the same GPU device so call sites written against the reference compile.
//===----------------------------------------------------------------------===//

#include <engine/check.hpp>
#include <engine/dtype.hpp>
#include <engine/half.hpp>

#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <functional>
#include <memory>
#include <numeric>
#include <ostream>
#include <sstream>
#include <string>
#include <utility>
#include <vector>

namespace engine {

enum class Device : std::uint8_t {
  CPU = 0,
  HIP = 1,
  CUDA = HIP,  // the reference's name for the GPU device
};

inline const char* device_name(Device d) {
  switch (d) {
    case Device::CPU: return "cpu";
    case Device::HIP: return "hip";
    default: return "<invalid>";
  }
}

inline std::ostream& operator<<(std::ostream& os, Device d) { return os << device_name(d); }

struct BorrowTag {};

class Storage {
 public:
  Storage(std::size_t bytes, Device device) : bytes_(bytes), device_(device) {
    if (bytes == 0) return;
    if (device == Device::CPU) {
      ptr_ = std::malloc(bytes);
      ENGINE_CHECK(ptr_ != nullptr, "host allocation failed");
    } else {
      ENGINE_ABI_CHECK(eng_malloc(&ptr_, bytes));
    }
  }

  Storage(void* data, std::size_t bytes, Device device, BorrowTag)
      : ptr_(data), bytes_(bytes), device_(device), owns_(false) {}

  ~Storage() {
    if (!owns_ || ptr_ == nullptr) return;
    if (device_ == Device::CPU) {
      std::free(ptr_);
    } else {
      (void)eng_free(ptr_);
    }
  }

  Storage(const Storage&) = delete;
  Storage& operator=(const Storage&) = delete;
  Storage(Storage&&) = delete;
  Storage& operator=(Storage&&) = delete;

  void* data() { return ptr_; }
  const void* data() const { return ptr_; }
  std::size_t bytes() const { return bytes_; }
  Device device() const { return device_; }
  bool owns() const { return owns_; }

 private:
  void* ptr_ = nullptr;
  std::size_t bytes_ = 0;
  Device device_ = Device::CPU;
  bool owns_ = true;
};

class Tensor {
 public:
  Tensor() = default;

  Tensor(std::vector<std::int64_t> shape, DType dtype, Device device)
      : shape_(std::move(shape)), dtype_(dtype), device_(device) {
    for (std::size_t i = 0; i < shape_.size(); ++i) {
      ENGINE_CHECK(shape_[i] >= 0, "Tensor: dimension " + std::to_string(i) + " is " +
                                       std::to_string(shape_[i]) + ", must be >= 0");
    }
    strides_ = contiguous_strides(shape_);
    storage_ = std::make_shared<Storage>(bytes_for(shape_, dtype_), device_);
  }

  static Tensor zeros(std::vector<std::int64_t> shape, DType dtype, Device device) {
    Tensor t(std::move(shape), dtype, device);
    const std::size_t bytes = t.nbytes();
    if (bytes == 0) return t;
    if (device == Device::CPU) {
      std::memset(t.storage_->data(), 0, bytes);
    } else {
      ENGINE_ABI_CHECK(eng_memset(t.storage_->data(), 0, bytes));
    }
    return t;
  }

  static Tensor from_blob(void* data, std::vector<std::int64_t> shape, DType dtype,
                          Device device) {
    ENGINE_CHECK(data != nullptr || shape.empty(),
                 "Tensor::from_blob: null data with non-empty shape");
    for (std::size_t i = 0; i < shape.size(); ++i) {
      ENGINE_CHECK(shape[i] >= 0, "Tensor::from_blob: dimension " + std::to_string(i) +
                                      " is " + std::to_string(shape[i]) + ", must be >= 0");
    }
    Tensor t;
    t.storage_ = std::make_shared<Storage>(data, bytes_for(shape, dtype), device, BorrowTag{});
    t.shape_ = std::move(shape);
    t.strides_ = contiguous_strides(t.shape_);
    t.dtype_ = dtype;
    t.device_ = device;
    return t;
  }

  /// Contiguous view of `shape` at `byte_offset` inside an existing Storage,
  /// sharing (and keeping alive) that Storage: many tensors aliasing one
  /// allocation, as a weight slab's tensors do.
  static Tensor view(std::shared_ptr<Storage> storage, std::int64_t byte_offset,
                     std::vector<std::int64_t> shape, DType dtype) {
    ENGINE_CHECK(storage != nullptr, "Tensor::view: storage is null");
    ENGINE_CHECK(!dtype_is_sub_byte(dtype), "Tensor::view: sub-byte dtypes are not supported");
    for (std::size_t i = 0; i < shape.size(); ++i) {
      ENGINE_CHECK(shape[i] >= 0, "Tensor::view: dimension " + std::to_string(i) + " is " +
                                      std::to_string(shape[i]) + ", must be >= 0");
    }
    const auto esz = static_cast<std::int64_t>(dtype_size(dtype));
    ENGINE_CHECK(byte_offset >= 0 && byte_offset % esz == 0,
                 "Tensor::view: byte offset " + std::to_string(byte_offset) +
                     " is not a non-negative multiple of the element size");
    const std::size_t bytes = bytes_for(shape, dtype);
    ENGINE_CHECK(static_cast<std::size_t>(byte_offset) + bytes <= storage->bytes(),
                 "Tensor::view: " + std::to_string(bytes) + " bytes at offset " +
                     std::to_string(byte_offset) + " overrun a storage of " +
                     std::to_string(storage->bytes()) + " bytes");
    Tensor t;
    t.device_ = storage->device();
    t.storage_ = std::move(storage);
    t.shape_ = std::move(shape);
    t.strides_ = contiguous_strides(t.shape_);
    t.offset_ = byte_offset / esz;
    t.dtype_ = dtype;
    return t;
  }

  // -- shape / layout ------------------------------------------------------
  const std::vector<std::int64_t>& shape() const { return shape_; }
  const std::vector<std::int64_t>& strides() const { return strides_; }
  std::int64_t dim() const { return static_cast<std::int64_t>(shape_.size()); }

  std::int64_t size(std::int64_t axis) const {
    if (axis < 0) axis += dim();
    ENGINE_CHECK(axis >= 0 && axis < dim(), "Tensor::size: axis " + std::to_string(axis) +
                                                " out of range for tensor with dim=" +
                                                std::to_string(dim()));
    return shape_[static_cast<std::size_t>(axis)];
  }

  std::int64_t numel() const { return defined() ? product(shape_) : 0; }

  std::size_t nbytes() const {
    const std::int64_t n = numel();
    return n > 0 ? dtype_storage_bytes(dtype_, static_cast<std::size_t>(n)) : 0;
  }

  DType dtype() const { return dtype_; }
  Device device() const { return device_; }
  bool defined() const { return storage_ != nullptr; }

  bool is_contiguous() const {
    std::int64_t expected = 1;
    for (std::int64_t i = dim() - 1; i >= 0; --i) {
      const auto d = static_cast<std::size_t>(i);
      if (shape_[d] == 0) return true;
      if (shape_[d] > 1 && strides_[d] != expected) return false;
      expected *= shape_[d];
    }
    return true;
  }

  // -- views -------------------------------------------------------------
  Tensor reshape(std::vector<std::int64_t> new_shape) const {
    ENGINE_CHECK(defined(), "Tensor::reshape called on undefined tensor");
    ENGINE_CHECK(is_contiguous(),
                 "Tensor::reshape requires a contiguous tensor. "
                 "Call .contiguous() first to pack the data.");
    const std::int64_t n = numel();
    std::int64_t infer = -1;
    std::int64_t known = 1;
    for (std::size_t i = 0; i < new_shape.size(); ++i) {
      if (new_shape[i] == -1) {
        ENGINE_CHECK(infer == -1, "Tensor::reshape: at most one dimension may be -1");
        infer = static_cast<std::int64_t>(i);
      } else {
        ENGINE_CHECK(new_shape[i] >= 0,
                     "Tensor::reshape: negative dimension " + std::to_string(new_shape[i]));
        known *= new_shape[i];
      }
    }
    if (infer >= 0) {
      ENGINE_CHECK(known > 0 && n % known == 0, "Tensor::reshape: cannot infer dimension for shape");
      new_shape[static_cast<std::size_t>(infer)] = n / known;
    }
    const std::int64_t new_n = product(new_shape);
    ENGINE_CHECK(new_n == n, "Tensor::reshape: cannot reshape " + std::to_string(n) +
                                 " elements into " + std::to_string(new_n));
    Tensor out = view_like();
    out.shape_ = std::move(new_shape);
    out.strides_ = contiguous_strides(out.shape_);
    return out;
  }

  Tensor permute(std::vector<std::int64_t> perm) const {
    ENGINE_CHECK(defined(), "Tensor::permute called on undefined tensor");
    ENGINE_CHECK(static_cast<std::int64_t>(perm.size()) == dim(),
                 "Tensor::permute: perm length " + std::to_string(perm.size()) + " != dim " +
                     std::to_string(dim()));
    std::vector<bool> seen(shape_.size(), false);
    Tensor out = view_like();
    for (std::size_t i = 0; i < perm.size(); ++i) {
      const std::int64_t p = perm[i];
      ENGINE_CHECK(p >= 0 && p < dim(), "Tensor::permute: axis " + std::to_string(p) +
                                            " out of range for dim=" + std::to_string(dim()));
      ENGINE_CHECK(!seen[static_cast<std::size_t>(p)],
                   "Tensor::permute: axis " + std::to_string(p) + " appears more than once");
      seen[static_cast<std::size_t>(p)] = true;
      out.shape_[i] = shape_[static_cast<std::size_t>(p)];
      out.strides_[i] = strides_[static_cast<std::size_t>(p)];
    }
    return out;
  }

  Tensor transpose(std::int64_t a, std::int64_t b) const {
    if (a < 0) a += dim();
    if (b < 0) b += dim();
    ENGINE_CHECK(a >= 0 && a < dim(), "Tensor::transpose: axis " + std::to_string(a) +
                                          " out of range for dim=" + std::to_string(dim()));
    ENGINE_CHECK(b >= 0 && b < dim(), "Tensor::transpose: axis " + std::to_string(b) +
                                          " out of range for dim=" + std::to_string(dim()));
    std::vector<std::int64_t> perm(shape_.size());
    std::iota(perm.begin(), perm.end(), std::int64_t{0});
    std::swap(perm[static_cast<std::size_t>(a)], perm[static_cast<std::size_t>(b)]);
    return permute(std::move(perm));
  }

  Tensor slice(std::int64_t axis, std::int64_t start, std::int64_t length) const {
    ENGINE_CHECK(defined(), "Tensor::slice called on undefined tensor");
    if (axis < 0) axis += dim();
    ENGINE_CHECK(axis >= 0 && axis < dim(), "Tensor::slice: axis " + std::to_string(axis) +
                                                " out of range for dim=" + std::to_string(dim()));
    ENGINE_CHECK(start >= 0, "Tensor::slice: start must be >= 0, got " + std::to_string(start));
    ENGINE_CHECK(length >= 0, "Tensor::slice: length must be >= 0, got " + std::to_string(length));
    const auto ax = static_cast<std::size_t>(axis);
    ENGINE_CHECK(start + length <= shape_[ax],
                 "Tensor::slice: start(" + std::to_string(start) + ") + length(" +
                     std::to_string(length) + ") > axis size(" + std::to_string(shape_[ax]) + ")");
    Tensor out = view_like();
    out.shape_[ax] = length;
    out.offset_ = offset_ + start * strides_[ax];
    return out;
  }

  // -- copies ------------------------------------------------------------
  Tensor contiguous() const {
    ENGINE_CHECK(defined(), "Tensor::contiguous called on undefined tensor");
    if (is_contiguous()) return *this;
    ENGINE_CHECK(device_ == Device::CPU,
                 "Tensor::contiguous on a non-contiguous GPU tensor is not supported. "
                 "Make views contiguous on CPU before transferring to the GPU.");
    Tensor out(shape_, dtype_, device_);
    const std::int64_t n = numel();
    if (n == 0) return out;
    const std::size_t esz = dtype_size(dtype_);
    const char* src = static_cast<const char*>(data());
    char* dst = static_cast<char*>(out.data());
    std::vector<std::int64_t> idx(shape_.size(), 0);
    std::int64_t src_off = 0;  // element offset of idx, kept incrementally
    for (std::int64_t flat = 0; flat < n; ++flat) {
      std::memcpy(dst + flat * static_cast<std::int64_t>(esz),
                  src + src_off * static_cast<std::int64_t>(esz), esz);
      for (std::int64_t d = dim() - 1; d >= 0; --d) {
        const auto k = static_cast<std::size_t>(d);
        ++idx[k];
        src_off += strides_[k];
        if (idx[k] < shape_[k]) break;
        src_off -= idx[k] * strides_[k];
        idx[k] = 0;
      }
    }
    return out;
  }

  Tensor clone() const {
    ENGINE_CHECK(defined(), "Tensor::clone called on undefined tensor");
    Tensor src = contiguous();
    Tensor out(src.shape_, src.dtype_, src.device_);
    const std::size_t bytes = src.nbytes();
    if (bytes == 0) return out;
    if (src.device_ == Device::CPU) {
      std::memcpy(out.storage_->data(), src.data(), bytes);
    } else {
      ENGINE_ABI_CHECK(eng_memcpy_d2d(out.storage_->data(), src.data(), bytes));
    }
    return out;
  }

  Tensor to(Device target) const {
    ENGINE_CHECK(defined(), "Tensor::to called on undefined tensor");
    if (device_ == target) return *this;
    ENGINE_CHECK(is_contiguous(),
                 "Tensor::to requires a contiguous tensor. Call .contiguous() first to pack the data.");
    Tensor out(shape_, dtype_, target);
    const std::size_t bytes = nbytes();
    if (bytes == 0) return out;
    if (device_ == Device::CPU) {
      ENGINE_ABI_CHECK(eng_memcpy_h2d(out.storage_->data(), data(), bytes));
    } else {
      ENGINE_ABI_CHECK(eng_memcpy_d2h(out.storage_->data(), data(), bytes));
    }
    return out;
  }

  // -- raw access --------------------------------------------------------
  void* data() {
    ENGINE_CHECK(defined(), "Tensor::data() called on undefined tensor");
    char* base = static_cast<char*>(storage_->data());
    if (dtype_is_sub_byte(dtype_)) {
      return base + static_cast<std::size_t>(offset_) * static_cast<std::size_t>(dtype_bits(dtype_)) / 8;
    }
    return base + offset_ * static_cast<std::int64_t>(dtype_size(dtype_));
  }
  const void* data() const { return const_cast<Tensor*>(this)->data(); }

  template <typename T>
  T* ptr(Device expect) {
    check_ptr(expect, sizeof(T));
    return static_cast<T*>(data());
  }
  template <typename T>
  const T* ptr(Device expect) const {
    check_ptr(expect, sizeof(T));
    return static_cast<const T*>(data());
  }

  const std::shared_ptr<Storage>& storage() const { return storage_; }
  std::int64_t storage_offset() const { return offset_; }

  std::string to_string() const {
    if (!defined()) return "Tensor(undefined)";
    std::ostringstream oss;
    oss << "Tensor(shape=[" << join(shape_) << "], strides=[" << join(strides_)
        << "], dtype=" << dtype_name(dtype_) << ", device=" << device_name(device_) << ", "
        << (is_contiguous() ? "contiguous" : "non-contiguous") << ")";
    return oss.str();
  }

 private:
  static std::int64_t product(const std::vector<std::int64_t>& v) {
    return std::accumulate(v.begin(), v.end(), std::int64_t{1}, std::multiplies<std::int64_t>());
  }

  static std::size_t bytes_for(const std::vector<std::int64_t>& shape, DType dtype) {
    const std::int64_t n = product(shape);
    return n > 0 ? dtype_storage_bytes(dtype, static_cast<std::size_t>(n)) : 0;
  }

  static std::vector<std::int64_t> contiguous_strides(const std::vector<std::int64_t>& shape) {
    std::vector<std::int64_t> s(shape.size());
    std::int64_t acc = 1;
    for (std::size_t i = shape.size(); i-- > 0;) {
      s[i] = acc;
      acc *= shape[i];
    }
    return s;
  }

  static std::string join(const std::vector<std::int64_t>& v) {
    std::ostringstream oss;
    for (std::size_t i = 0; i < v.size(); ++i) oss << (i ? "," : "") << v[i];
    return oss.str();
  }

  Tensor view_like() const {
    Tensor out;
    out.storage_ = storage_;
    out.shape_ = shape_;
    out.strides_ = strides_;
    out.offset_ = offset_;
    out.dtype_ = dtype_;
    out.device_ = device_;
    return out;
  }

  void check_ptr(Device expect, std::size_t elem) const {
    ENGINE_CHECK(device_ == expect, "Tensor::ptr: expected device " +
                                        std::string(device_name(expect)) + " but tensor is on " +
                                        std::string(device_name(device_)));
    if (!dtype_is_sub_byte(dtype_)) {
      ENGINE_CHECK(elem == dtype_size(dtype_),
                   "Tensor::ptr: sizeof(T)=" + std::to_string(elem) +
                       " does not match dtype element size " + std::to_string(dtype_size(dtype_)));
    }
  }

  std::shared_ptr<Storage> storage_;
  std::vector<std::int64_t> shape_;
  std::vector<std::int64_t> strides_;
  std::int64_t offset_ = 0;  // in elements
  DType dtype_ = DType::F32;
  Device device_ = Device::CPU;
};

}  // namespace engine
