#pragma once
//===----------------------------------------------------------------------===//
// engine/half.hpp -- IEEE-754 binary16 storage type and host conversions.
//
// Same names as the reference (include/engine/half.hpp:27-105): engine::half,
// half_to_float, float_to_half, float_to_half_bits, half_bits_to_float. One
// deliberate difference: float -> half rounds to nearest, ties to even, in
// every build. The reference's non-CUDA host path truncates the mantissa
// (half.hpp:44-61), which would make host-prepared fp16 weights differ from
// device-rounded ones; RNE is what IEEE-754, NumPy's float16 and the GPU's
// conversion instruction all do.
//
// The type is a plain 16-bit struct on host and device, so buffers of it can
// be handed to the C-ABI (eng_half*) without conversion.
//===----------------------------------------------------------------------===//

#include <cstdint>
#include <cstring>
#include <ostream>

namespace engine {

struct half {
  std::uint16_t u = 0;

  half() = default;
  constexpr explicit half(std::uint16_t raw) : u(raw) {}
};

static_assert(sizeof(half) == 2, "engine::half must be 16 bits");

/// float -> binary16 bits, round to nearest even. Overflow gives +-inf, NaN stays
/// NaN (quiet bit set, top payload bits kept), underflow goes through the
/// subnormals to +-0.
inline std::uint16_t float_to_half_bits(float f) {
  std::uint32_t x;
  std::memcpy(&x, &f, sizeof(x));
  const std::uint32_t sign = (x >> 16) & 0x8000u;
  const std::uint32_t ax = x & 0x7fffffffu;

  if (ax >= 0x7f800000u) {  // inf or NaN
    if (ax == 0x7f800000u) return static_cast<std::uint16_t>(sign | 0x7c00u);
    return static_cast<std::uint16_t>(sign | 0x7e00u | ((ax >> 13) & 0x03ffu));
  }
  // 65520 = 0x477ff000 is the midpoint between the largest half (65504) and
  // 2^16; the tie goes to the even neighbour, 2^16, which is out of range.
  if (ax >= 0x477ff000u) return static_cast<std::uint16_t>(sign | 0x7c00u);

  if (ax < 0x38800000u) {  // below 2^-14: half subnormal m * 2^-24 or zero
    // At or below 2^-25 (half of the smallest subnormal) the value rounds to 0.
    if (ax <= 0x33000000u) return static_cast<std::uint16_t>(sign);
    const std::uint32_t exp = ax >> 23;                        // 102 .. 112
    const std::uint32_t mant = (ax & 0x007fffffu) | 0x00800000u;
    const std::uint32_t shift = 126u - exp;                    // 14 .. 24
    std::uint32_t m = mant >> shift;
    const std::uint32_t rem = mant & ((1u << shift) - 1u);
    const std::uint32_t halfway = 1u << (shift - 1u);
    if (rem > halfway || (rem == halfway && (m & 1u))) ++m;   // may carry to 0x400
    return static_cast<std::uint16_t>(sign | m);
  }

  // Normal range: rebias the exponent, keep 10 mantissa bits, round the 13 dropped.
  std::uint32_t h = (((ax >> 23) - 112u) << 10) | ((ax >> 13) & 0x03ffu);
  const std::uint32_t rem = ax & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) ++h;     // carry may bump exponent
  return static_cast<std::uint16_t>(sign | h);
}

/// binary16 bits -> float (exact).
inline float half_bits_to_float(std::uint16_t h) {
  const std::uint32_t sign = (static_cast<std::uint32_t>(h) & 0x8000u) << 16;
  const std::uint32_t exp = (h >> 10) & 0x1fu;
  std::uint32_t mant = h & 0x03ffu;
  std::uint32_t out;
  if (exp == 0) {
    if (mant == 0) {
      out = sign;
    } else {  // subnormal: normalise
      std::uint32_t e = 113;  // 127 - 14
      while ((mant & 0x0400u) == 0) {
        mant <<= 1;
        --e;
      }
      out = sign | (e << 23) | ((mant & 0x03ffu) << 13);
    }
  } else if (exp == 31) {
    out = sign | 0x7f800000u | (mant << 13);
  } else {
    out = sign | ((exp + 112u) << 23) | (mant << 13);
  }
  float f;
  std::memcpy(&f, &out, sizeof(f));
  return f;
}

inline float half_to_float(half h) { return half_bits_to_float(h.u); }
inline half float_to_half(float f) { return half(float_to_half_bits(f)); }

inline bool operator==(half a, half b) { return a.u == b.u; }
inline bool operator!=(half a, half b) { return a.u != b.u; }
inline bool operator<(half a, half b) { return half_to_float(a) < half_to_float(b); }
inline bool operator<=(half a, half b) { return half_to_float(a) <= half_to_float(b); }
inline bool operator>(half a, half b) { return half_to_float(a) > half_to_float(b); }
inline bool operator>=(half a, half b) { return half_to_float(a) >= half_to_float(b); }

inline std::ostream& operator<<(std::ostream& os, half h) { return os << half_to_float(h); }

}  // namespace engine
