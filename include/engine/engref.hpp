#pragma once
//===----------------------------------------------------------------------===//
// engine/engref.hpp -- ENGREF01 tensor files and device weight slabs.
//
// EngrefFile keeps the interface of the reference's golden reader
// (tests/golden.hpp:48-72: load / try_load / at / has / names / size, a
// bounds-checked dim()) over the library's memory-mapped reader
// (eng_engref_*): tensors are not copied on open, keep their dtype (f32, f16
// at native size, f64) and expose their bytes in place; floats() converts to
// float32 for the reference's `data` use. WeightSlab is the on-disk-to-HBM
// step of the reference's planned mmap weight loader (README.md:247): one
// device Storage holding every tensor of a file at 256-byte aligned offsets,
// handing out Tensor views that alias it and keep it alive.
//===----------------------------------------------------------------------===//

#include <engine/check.hpp>
#include <engine/dtype.hpp>
#include <engine/half.hpp>
#include <engine/tensor.hpp>

#include <algorithm>
#include <cstdint>
#include <cstring>
#include <memory>
#include <string>
#include <vector>

namespace engine {

struct EngrefTensor {
  std::string name;
  std::int32_t code = ENG_ENGREF_F32;  ///< ENG_ENGREF_F32 / _F16 / _F64
  std::vector<std::int64_t> shape;
  std::int64_t nbytes = 0;
  /// The mapped bytes (little-endian, maybe unaligned); valid while an
  /// EngrefFile or WeightSlab of this file is alive (they share the mapping).
  const void* host = nullptr;
  std::int64_t slab_offset = 0;

  std::int64_t numel() const {
    std::int64_t n = 1;
    for (auto d : shape) n *= d;
    return n;
  }

  /// shape[axis]; throws on a bad axis (reference GoldenTensor::dim).
  std::int64_t dim(std::size_t axis) const {
    ENGINE_CHECK(axis < shape.size(), "EngrefTensor::dim(): axis " + std::to_string(axis) +
                                          " out of range for a " +
                                          std::to_string(shape.size()) + "-d tensor");
    return shape[axis];
  }

  /// The Tensor dtype of the stored elements (f64 has none).
  DType dtype() const {
    ENGINE_CHECK(code != ENG_ENGREF_F64, "engref tensor '" + name + "' is float64, which no Tensor dtype holds");
    return code == ENG_ENGREF_F16 ? DType::F16 : DType::F32;
  }

  /// The elements converted to float32 (f16 exactly, f64 rounded).
  std::vector<float> floats() const {
    const auto n = static_cast<std::size_t>(numel());
    std::vector<float> out(n);
    const auto* p = static_cast<const unsigned char*>(host);
    for (std::size_t i = 0; i < n; ++i) {
      if (code == ENG_ENGREF_F32) {
        std::memcpy(&out[i], p + 4 * i, 4);
      } else if (code == ENG_ENGREF_F16) {
        std::uint16_t bits;
        std::memcpy(&bits, p + 2 * i, 2);
        out[i] = half_bits_to_float(bits);
      } else {
        double d;
        std::memcpy(&d, p + 8 * i, 8);
        out[i] = static_cast<float>(d);
      }
    }
    return out;
  }
};

class EngrefFile {
 public:
  EngrefFile() = default;

  /// Maps and validates `path`; throws EngineError with the reader's message.
  static EngrefFile load(const std::string& path) {
    EngrefFile f;
    eng_engref h = nullptr;
    ENGINE_ABI_CHECK(eng_engref_open(path.c_str(), &h));
    f.handle_.reset(h, [](eng_engref p) { (void)eng_engref_close(p); });
    std::int32_t n = 0;
    ENGINE_ABI_CHECK(eng_engref_count(h, &n));
    for (std::int32_t i = 0; i < n; ++i) {
      EngrefTensor t;
      const char* name = nullptr;
      std::int32_t ndim = 0;
      const std::int64_t* dims = nullptr;
      ENGINE_ABI_CHECK(eng_engref_tensor(h, i, &name, &t.code, &ndim, &dims, &t.nbytes,
                                         &t.host, &t.slab_offset));
      t.name = name;
      t.shape.assign(dims, dims + ndim);
      f.tensors_.push_back(std::move(t));
    }
    return f;
  }

  /// false (with `error` set) instead of throwing.
  static bool try_load(const std::string& path, EngrefFile& out, std::string& error) {
    try {
      out = load(path);
      return true;
    } catch (const std::exception& e) {
      error = e.what();
      return false;
    }
  }

  /// Throws if `name` is absent, listing the names present.
  const EngrefTensor& at(const std::string& name) const {
    std::int32_t i = 0;
    ENGINE_ABI_CHECK(eng_engref_find(handle(), name.c_str(), &i));
    return tensors_[static_cast<std::size_t>(i)];
  }

  bool has(const std::string& name) const {
    for (const auto& t : tensors_) {
      if (t.name == name) return true;
    }
    return false;
  }

  /// Names in sorted order (the reference reader keeps a std::map).
  std::vector<std::string> names() const {
    std::vector<std::string> out;
    for (const auto& t : tensors_) out.push_back(t.name);
    std::sort(out.begin(), out.end());
    return out;
  }

  std::size_t size() const { return tensors_.size(); }
  const std::vector<EngrefTensor>& tensors() const { return tensors_; }

  std::int64_t slab_bytes() const {
    std::int64_t b = 0;
    ENGINE_ABI_CHECK(eng_engref_slab_bytes(handle(), &b));
    return b;
  }

  eng_engref handle() const {
    ENGINE_CHECK(handle_ != nullptr, "EngrefFile: no file loaded");
    return handle_.get();
  }

 private:
  std::shared_ptr<eng_engref_s> handle_;
  std::vector<EngrefTensor> tensors_;
};

class WeightSlab {
 public:
  /// Allocates one device Storage for every tensor of `file` and uploads
  /// them on `stream` (returns when the copies are complete).
  static WeightSlab upload(const EngrefFile& file, eng_stream stream = nullptr) {
    WeightSlab s;
    s.file_ = file;
    const std::int64_t bytes = file.slab_bytes();
    s.storage_ = std::make_shared<Storage>(static_cast<std::size_t>(bytes), Device::HIP);
    ENGINE_ABI_CHECK(eng_engref_upload(file.handle(), s.storage_->data(), bytes, stream));
    return s;
  }

  /// A device Tensor aliasing the slab (f32 / f16 tensors).
  Tensor tensor(const std::string& name) const {
    const EngrefTensor& t = file_.at(name);
    return Tensor::view(storage_, t.slab_offset, t.shape, t.dtype());
  }

  /// Device address of a tensor's first byte (any dtype).
  const void* data(const std::string& name) const {
    return static_cast<const char*>(storage_->data()) + file_.at(name).slab_offset;
  }

  std::size_t bytes() const { return storage_ ? storage_->bytes() : 0; }
  const std::shared_ptr<Storage>& storage() const { return storage_; }

 private:
  EngrefFile file_;
  std::shared_ptr<Storage> storage_;
};

}  // namespace engine
