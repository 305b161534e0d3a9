#pragma once
//===----------------------------------------------------------------------===//
// engine/dtype.hpp -- element types a Tensor can hold.
//
// Same enumeration, values and helper names as the reference
// (include/engine/dtype.hpp:19-125), because Tensor and the golden tooling
// exchange these codes. Sizes are expressed in bits so the packed 4-bit type
// has an exact answer; byte-size queries on sub-byte types are errors.
//===----------------------------------------------------------------------===//

#include <engine/check.hpp>

#include <cstddef>
#include <cstdint>
#include <ostream>

namespace engine {

enum class DType : std::uint8_t {
  F32 = 0,
  F16 = 1,
  BF16 = 2,
  I32 = 3,
  I8 = 4,
  U8 = 5,
  I4 = 6,  ///< two per byte, never addressed individually
  COUNT = 7
};

constexpr int dtype_bits(DType dt) {
  return dt == DType::F32 || dt == DType::I32   ? 32
         : dt == DType::F16 || dt == DType::BF16 ? 16
         : dt == DType::I8 || dt == DType::U8    ? 8
         : dt == DType::I4                       ? 4
                                                 : 0;
}

constexpr bool dtype_is_sub_byte(DType dt) { return dtype_bits(dt) < 8; }

constexpr bool dtype_is_float(DType dt) {
  return dt == DType::F32 || dt == DType::F16 || dt == DType::BF16;
}

constexpr bool dtype_is_quantised(DType dt) { return dt == DType::I8 || dt == DType::I4; }

/// Bytes per element; an error for sub-byte types (use dtype_storage_bytes).
inline std::size_t dtype_size(DType dt) {
  ENGINE_CHECK(!dtype_is_sub_byte(dt),
               "dtype_size() is undefined for sub-byte types; use dtype_storage_bytes()");
  const int bits = dtype_bits(dt);
  ENGINE_CHECK(bits > 0, "unknown DType passed to dtype_size()");
  return static_cast<std::size_t>(bits / 8);
}

/// Bytes holding n elements, rounded up to whole bytes (works for I4).
inline std::size_t dtype_storage_bytes(DType dt, std::size_t n) {
  const int bits = dtype_bits(dt);
  ENGINE_CHECK(bits > 0, "unknown DType passed to dtype_storage_bytes()");
  return (n * static_cast<std::size_t>(bits) + 7u) / 8u;
}

inline const char* dtype_name(DType dt) {
  switch (dt) {
    case DType::F32: return "f32";
    case DType::F16: return "f16";
    case DType::BF16: return "bf16";
    case DType::I32: return "i32";
    case DType::I8: return "i8";
    case DType::U8: return "u8";
    case DType::I4: return "i4";
    default: return "<invalid>";
  }
}

inline std::ostream& operator<<(std::ostream& os, DType dt) { return os << dtype_name(dt); }

/// Elements per quantisation block (GGUF Q4_0 / Q8_0 families).
constexpr int kQuantBlockSize = 32;

/// Bytes of one quantised block including its fp16 scale.
inline std::size_t quant_block_bytes(DType dt) {
  ENGINE_CHECK(dtype_is_quantised(dt), "quant_block_bytes() requires a quantised DType");
  return dtype_storage_bytes(dt, static_cast<std::size_t>(kQuantBlockSize)) +
         sizeof(std::uint16_t);
}

/// Bits per weight including the scale overhead.
inline double quant_effective_bits(DType dt) {
  return 8.0 * static_cast<double>(quant_block_bytes(dt)) / static_cast<double>(kQuantBlockSize);
}

}  // namespace engine
