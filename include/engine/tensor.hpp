#pragma once
//===----------------------------------------------------------------------===//
// engine/tensor.hpp -- Storage (owning or borrowed bytes) and Tensor (views).
//
// The contract is the reference's Tensor/Storage interface
// (include/engine/tensor.hpp:50-195) as its tests pin it
// (tests/test_tensor.cpp:70-625); the implementation here is header-only and
// allocates device bytes through the engine's C-ABI (eng_malloc / eng_free).
//
//   * Storage owns `bytes` on one device or borrows a caller's pointer that it
//     never frees; a zero-byte Storage holds no pointer.
//   * Tensor = Layout (sizes, strides in elements, element offset) + dtype +
//     a shared Storage. reshape / permute / transpose / slice only edit the
//     layout and share the Storage (a view keeps it alive); contiguous /
//     clone / to copy bytes.
//   * numel() of an undefined tensor is 0 and of a rank-0 tensor 1; a size-0
//     axis makes the tensor empty, and an empty tensor counts as contiguous.
//   * reshape needs a contiguous view and infers at most one -1.
//   * A non-contiguous GPU view cannot be packed on the device: contiguous()
//     and to() say so and name the fix (pack on the host first).
//   * ptr<T>(device) checks the device first, then sizeof(T) against the
//     element size.
// Device numbering matches the C-ABI (ENG_DEVICE_CPU = 0, ENG_DEVICE_GPU = 1);
// Device::CUDA is another name for the GPU so reference call sites compile.
//===----------------------------------------------------------------------===//

#include <engine/check.hpp>
#include <engine/dtype.hpp>
#include <engine/half.hpp>

#include <algorithm>
#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <memory>
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
  return d == Device::CPU ? "cpu" : d == Device::HIP ? "hip" : "<invalid>";
}

inline std::ostream& operator<<(std::ostream& os, Device d) { return os << device_name(d); }

struct BorrowTag {};

/// A block of bytes on one device. Owning storage releases its block with the
/// matching deallocator; borrowed storage (from_blob, mapped files) never does.
class Storage {
 public:
  /// Owning: host blocks are 256-byte aligned (like the device allocator's), so
  /// vector loads over host tensors never straddle an alignment boundary.
  Storage(std::size_t bytes, Device device) : bytes_(bytes), device_(device) {
    if (bytes == 0) return;
    if (device == Device::CPU) {
      const std::size_t rounded = (bytes + kHostAlign - 1) / kHostAlign * kHostAlign;
      ptr_ = std::aligned_alloc(kHostAlign, rounded);
      ENGINE_CHECK(ptr_ != nullptr, "Storage: host allocation of " + std::to_string(bytes) +
                                        " bytes failed");
      release_ = &release_host;
    } else {
      ENGINE_ABI_CHECK(eng_malloc(&ptr_, bytes));
      release_ = &release_device;
    }
  }

  /// Borrowing: `data` stays the caller's.
  Storage(void* data, std::size_t bytes, Device device, BorrowTag)
      : ptr_(data), bytes_(bytes), device_(device) {}

  ~Storage() {
    if (release_ != nullptr && ptr_ != nullptr) release_(ptr_);
  }

  Storage(const Storage&) = delete;
  Storage& operator=(const Storage&) = delete;
  Storage(Storage&&) = delete;
  Storage& operator=(Storage&&) = delete;

  void* data() { return ptr_; }
  const void* data() const { return ptr_; }
  std::size_t bytes() const { return bytes_; }
  Device device() const { return device_; }
  bool owns() const { return release_ != nullptr; }

 private:
  static constexpr std::size_t kHostAlign = 256;
  static void release_host(void* p) { std::free(p); }
  static void release_device(void* p) { (void)eng_free(p); }  // destructors do not throw

  void* ptr_ = nullptr;
  std::size_t bytes_ = 0;
  Device device_ = Device::CPU;
  void (*release_)(void*) = nullptr;  // null: borrowed
};

class Tensor {
 public:
  using Dims = std::vector<std::int64_t>;

  Tensor() = default;

  /// Allocates row-major storage for `shape`; the bytes are left uninitialised.
  Tensor(Dims shape, DType dtype, Device device) : dtype_(dtype), device_(device) {
    require_sizes(shape, "Tensor");
    sizes_ = std::move(shape);
    strides_ = row_major(sizes_);
    storage_ = std::make_shared<Storage>(storage_bytes(sizes_, dtype_), device_);
  }

  static Tensor zeros(Dims shape, DType dtype, Device device) {
    Tensor t(std::move(shape), dtype, device);
    fill_bytes(t, 0);
    return t;
  }

  /// A contiguous tensor over caller memory that it never frees.
  static Tensor from_blob(void* data, Dims shape, DType dtype, Device device) {
    require_sizes(shape, "Tensor::from_blob");
    const std::size_t bytes = storage_bytes(shape, dtype);
    ENGINE_CHECK(data != nullptr || bytes == 0,
                 "Tensor::from_blob: data is null but the shape holds " + std::to_string(bytes) +
                     " bytes");
    auto s = std::make_shared<Storage>(data, bytes, device, BorrowTag{});
    return Tensor(std::move(s), std::move(shape), 0, dtype);
  }

  /// Contiguous view of `shape` at `byte_offset` inside an existing Storage,
  /// sharing (and keeping alive) that Storage: many tensors aliasing one
  /// allocation, as a weight slab's tensors do.
  static Tensor view(std::shared_ptr<Storage> storage, std::int64_t byte_offset, Dims shape,
                     DType dtype) {
    ENGINE_CHECK(storage != nullptr, "Tensor::view: storage is null");
    ENGINE_CHECK(!dtype_is_sub_byte(dtype), "Tensor::view: sub-byte dtypes are not supported");
    require_sizes(shape, "Tensor::view");
    const auto elem = static_cast<std::int64_t>(dtype_size(dtype));
    ENGINE_CHECK(byte_offset >= 0 && byte_offset % elem == 0,
                 "Tensor::view: byte offset " + std::to_string(byte_offset) +
                     " is not a non-negative multiple of the element size");
    const std::size_t need = static_cast<std::size_t>(byte_offset) + storage_bytes(shape, dtype);
    ENGINE_CHECK(need <= storage->bytes(),
                 "Tensor::view: " + std::to_string(need - static_cast<std::size_t>(byte_offset)) +
                     " bytes at offset " + std::to_string(byte_offset) + " overrun a storage of " +
                     std::to_string(storage->bytes()) + " bytes");
    return Tensor(std::move(storage), std::move(shape), byte_offset / elem, dtype);
  }

  // -- metadata ------------------------------------------------------------
  const Dims& shape() const { return sizes_; }
  const Dims& strides() const { return strides_; }
  std::int64_t dim() const { return static_cast<std::int64_t>(sizes_.size()); }
  std::int64_t size(std::int64_t axis) const { return sizes_[wrap_axis(axis, "size")]; }
  std::int64_t numel() const { return defined() ? count(sizes_) : 0; }
  std::size_t nbytes() const { return defined() ? storage_bytes(sizes_, dtype_) : 0; }
  DType dtype() const { return dtype_; }
  Device device() const { return device_; }
  bool defined() const { return storage_ != nullptr; }
  const std::shared_ptr<Storage>& storage() const { return storage_; }
  std::int64_t storage_offset() const { return offset_; }

  /// Row-major packed: every axis longer than 1 has the stride a freshly
  /// allocated tensor of this shape would have. Empty tensors qualify.
  bool is_contiguous() const {
    if (numel() == 0) return true;
    const Dims packed = row_major(sizes_);
    for (std::size_t i = 0; i < sizes_.size(); ++i) {
      if (sizes_[i] != 1 && strides_[i] != packed[i]) return false;
    }
    return true;
  }

  // -- views (layout edits, shared storage) -------------------------------
  Tensor reshape(Dims dims) const {
    require_defined("reshape");
    ENGINE_CHECK(is_contiguous(),
                 "Tensor::reshape: this view is not contiguous; call .contiguous() to pack it "
                 "into a new tensor first");
    const auto holes = std::count(dims.begin(), dims.end(), std::int64_t{-1});
    ENGINE_CHECK(holes <= 1, "Tensor::reshape: at most one dimension may be -1, got " +
                                 std::to_string(holes));
    std::int64_t known = 1;
    for (const std::int64_t d : dims) {
      if (d == -1) continue;
      ENGINE_CHECK(d >= 0, "Tensor::reshape: dimension " + std::to_string(d) + " is negative");
      known *= d;
    }
    const std::int64_t n = numel();
    if (holes == 1) {
      ENGINE_CHECK(known > 0 && n % known == 0,
                   "Tensor::reshape: cannot infer the -1 dimension: " + std::to_string(n) +
                       " elements are not a multiple of " + std::to_string(known));
      *std::find(dims.begin(), dims.end(), std::int64_t{-1}) = n / known;
    } else {
      ENGINE_CHECK(known == n, "Tensor::reshape: cannot reshape " + std::to_string(n) +
                                   " elements into a shape of " + std::to_string(known));
    }
    Tensor out = *this;
    out.strides_ = row_major(dims);
    out.sizes_ = std::move(dims);
    return out;
  }

  Tensor permute(const Dims& order) const {
    require_defined("permute");
    ENGINE_CHECK(static_cast<std::int64_t>(order.size()) == dim(),
                 "Tensor::permute: perm length " + std::to_string(order.size()) +
                     " does not match the tensor's " + std::to_string(dim()) + " axes");
    // A permutation of 0..dim-1 is exactly a list whose sorted copy is 0..dim-1.
    Dims sorted = order;
    std::sort(sorted.begin(), sorted.end());
    for (std::size_t i = 0; i < sorted.size(); ++i) {
      ENGINE_CHECK(sorted[i] == static_cast<std::int64_t>(i),
                   "Tensor::permute: [" + join(order) + "] is not a permutation of the axes 0.." +
                       std::to_string(dim() - 1) + " (an axis is out of range or appears more "
                       "than once)");
    }
    Tensor out = *this;
    for (std::size_t i = 0; i < order.size(); ++i) {
      out.sizes_[i] = sizes_[static_cast<std::size_t>(order[i])];
      out.strides_[i] = strides_[static_cast<std::size_t>(order[i])];
    }
    return out;
  }

  Tensor transpose(std::int64_t a, std::int64_t b) const {
    require_defined("transpose");
    const std::size_t i = wrap_axis(a, "transpose");
    const std::size_t j = wrap_axis(b, "transpose");
    Tensor out = *this;
    std::swap(out.sizes_[i], out.sizes_[j]);
    std::swap(out.strides_[i], out.strides_[j]);
    return out;
  }

  /// Elements [start, start + length) of `axis`; strides are unchanged and the
  /// offset accumulates, so slices of slices compose.
  Tensor slice(std::int64_t axis, std::int64_t start, std::int64_t length) const {
    require_defined("slice");
    const std::size_t ax = wrap_axis(axis, "slice");
    ENGINE_CHECK(start >= 0 && length >= 0,
                 "Tensor::slice: start (" + std::to_string(start) + ") and length (" +
                     std::to_string(length) + ") must be >= 0");
    ENGINE_CHECK(start + length <= sizes_[ax],
                 "Tensor::slice: [" + std::to_string(start) + ", " +
                     std::to_string(start + length) + ") runs past axis " + std::to_string(ax) +
                     " of axis size " + std::to_string(sizes_[ax]));
    Tensor out = *this;
    out.sizes_[ax] = length;
    out.offset_ += start * strides_[ax];
    return out;
  }

  // -- copies ------------------------------------------------------------
  /// This tensor if it is already packed; otherwise a packed copy (host only).
  Tensor contiguous() const {
    require_defined("contiguous");
    if (is_contiguous()) return *this;
    ENGINE_CHECK(device_ == Device::CPU,
                 "Tensor::contiguous: a non-contiguous GPU view cannot be packed on the device; "
                 "make the view contiguous on the CPU (Device::CPU) before moving it to the GPU");
    Tensor out(sizes_, dtype_, device_);
    pack_host_into(out);
    return out;
  }

  /// Always a new, packed allocation on the same device.
  Tensor clone() const {
    require_defined("clone");
    if (!is_contiguous()) return contiguous();  // contiguous() already allocated
    Tensor out(sizes_, dtype_, device_);
    copy_bytes(out.data(), data(), nbytes(), device_, device_);
    return out;
  }

  /// This tensor on `target`; the same tensor when it is already there.
  Tensor to(Device target) const {
    require_defined("to");
    if (target == device_) return *this;
    ENGINE_CHECK(is_contiguous(),
                 "Tensor::to: the view is not contiguous; call .contiguous() (on the CPU) "
                 "before copying it to another device");
    Tensor out(sizes_, dtype_, target);
    copy_bytes(out.data(), data(), nbytes(), target, device_);
    return out;
  }

  // -- raw access --------------------------------------------------------
  void* data() {
    require_defined("data");
    return static_cast<char*>(storage_->data()) + offset_bytes(offset_, dtype_);
  }
  const void* data() const { return const_cast<Tensor*>(this)->data(); }

  template <typename T>
  T* ptr(Device expect) {
    check_access(expect, sizeof(T));
    return static_cast<T*>(data());
  }
  template <typename T>
  const T* ptr(Device expect) const {
    check_access(expect, sizeof(T));
    return static_cast<const T*>(data());
  }

  std::string to_string() const {
    if (!defined()) return "Tensor(undefined)";
    std::ostringstream os;
    os << "Tensor(" << dtype_name(dtype_) << " on " << device_name(device_) << ", shape ["
       << join(sizes_) << "], strides [" << join(strides_) << "], offset " << offset_ << ", "
       << (is_contiguous() ? "contiguous" : "non-contiguous") << ")";
    return os.str();
  }

 private:
  Tensor(std::shared_ptr<Storage> storage, Dims sizes, std::int64_t offset, DType dtype)
      : storage_(std::move(storage)), sizes_(std::move(sizes)), offset_(offset), dtype_(dtype) {
    device_ = storage_->device();
    strides_ = row_major(sizes_);
  }

  static std::int64_t count(const Dims& sizes) {
    std::int64_t n = 1;
    for (const std::int64_t s : sizes) n *= s;
    return n;
  }

  static std::size_t storage_bytes(const Dims& sizes, DType dtype) {
    const std::int64_t n = count(sizes);
    return n > 0 ? dtype_storage_bytes(dtype, static_cast<std::size_t>(n)) : 0;
  }

  /// Byte position of element `elem` (sub-byte types pack several per byte).
  static std::size_t offset_bytes(std::int64_t elem, DType dtype) {
    return static_cast<std::size_t>(elem) * static_cast<std::size_t>(dtype_bits(dtype)) / 8u;
  }

  static Dims row_major(const Dims& sizes) {
    Dims strides(sizes.size(), 1);
    for (std::size_t i = sizes.size(); i > 1; --i) strides[i - 2] = strides[i - 1] * sizes[i - 1];
    return strides;
  }

  static void require_sizes(const Dims& sizes, const char* who) {
    for (std::size_t i = 0; i < sizes.size(); ++i) {
      ENGINE_CHECK(sizes[i] >= 0, std::string(who) + ": dimension " + std::to_string(i) +
                                      " is " + std::to_string(sizes[i]) + ", must be >= 0");
    }
  }

  static std::string join(const Dims& v) {
    std::string s;
    for (std::size_t i = 0; i < v.size(); ++i) s += (i ? ", " : "") + std::to_string(v[i]);
    return s;
  }

  static void fill_bytes(Tensor& t, int value) {
    const std::size_t bytes = t.nbytes();
    if (bytes == 0) return;
    if (t.device_ == Device::CPU) {
      std::memset(t.data(), value, bytes);
    } else {
      ENGINE_ABI_CHECK(eng_memset(t.data(), value, bytes));
    }
  }

  /// `bytes` from src (on `from`) to dst (on `to`), synchronously.
  static void copy_bytes(void* dst, const void* src, std::size_t bytes, Device to, Device from) {
    if (bytes == 0) return;
    if (to == Device::CPU && from == Device::CPU) {
      std::memcpy(dst, src, bytes);
    } else if (from == Device::CPU) {
      ENGINE_ABI_CHECK(eng_memcpy_h2d(dst, src, bytes));
    } else if (to == Device::CPU) {
      ENGINE_ABI_CHECK(eng_memcpy_d2h(dst, src, bytes));
    } else {
      ENGINE_ABI_CHECK(eng_memcpy_d2d(dst, src, bytes));
    }
  }

  std::size_t wrap_axis(std::int64_t axis, const char* op) const {
    const std::int64_t a = axis < 0 ? axis + dim() : axis;
    ENGINE_CHECK(a >= 0 && a < dim(), std::string("Tensor::") + op + ": axis " +
                                          std::to_string(axis) + " is out of range for a tensor "
                                          "with dim=" + std::to_string(dim()));
    return static_cast<std::size_t>(a);
  }

  void require_defined(const char* op) const {
    ENGINE_CHECK(defined(), std::string("Tensor::") + op + " called on an undefined tensor");
  }

  void check_access(Device expect, std::size_t elem) const {
    ENGINE_CHECK(device_ == expect, "Tensor::ptr: expected device " +
                                        std::string(device_name(expect)) + " but tensor is on " +
                                        std::string(device_name(device_)));
    ENGINE_CHECK(dtype_is_sub_byte(dtype_) || elem == dtype_size(dtype_),
                 "Tensor::ptr: sizeof(T) = " + std::to_string(elem) +
                     " does not match the element size of " + dtype_name(dtype_));
  }

  /// Packs this (host, strided) view into `out` (host, packed, same shape):
  /// whole rows of the innermost axis at a time, one memcpy per row when that
  /// axis is unit-stride. Sub-byte dtypes have no addressable elements and are
  /// refused.
  void pack_host_into(Tensor& out) const {
    ENGINE_CHECK(!dtype_is_sub_byte(dtype_),
                 "Tensor::contiguous: strided sub-byte tensors cannot be packed");
    if (numel() == 0) return;
    const std::size_t elem = dtype_size(dtype_);
    const char* src = static_cast<const char*>(storage_->data());
    char* dst = static_cast<char*>(out.data());
    copy_axis(0, offset_, src, dst, elem);
  }

  // Copies the sub-block of axes [axis, dim) whose first element is at element
  // `at` of the storage to `dst`; returns the end of what it wrote.
  char* copy_axis(std::size_t axis, std::int64_t at, const char* src, char* dst,
                  std::size_t elem) const {
    const std::int64_t n = sizes_[axis];
    const std::int64_t step = strides_[axis];
    if (axis + 1 == sizes_.size()) {
      if (step == 1) {
        const std::size_t row = static_cast<std::size_t>(n) * elem;
        std::memcpy(dst, src + static_cast<std::size_t>(at) * elem, row);
        return dst + row;
      }
      for (std::int64_t i = 0; i < n; ++i, dst += elem) {
        std::memcpy(dst, src + static_cast<std::size_t>(at + i * step) * elem, elem);
      }
      return dst;
    }
    for (std::int64_t i = 0; i < n; ++i) dst = copy_axis(axis + 1, at + i * step, src, dst, elem);
    return dst;
  }

  std::shared_ptr<Storage> storage_;
  Dims sizes_;
  Dims strides_;
  std::int64_t offset_ = 0;  // in elements
  DType dtype_ = DType::F32;
  Device device_ = Device::CPU;
};

}  // namespace engine
