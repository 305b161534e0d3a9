// half_host.cpp -- host fp16 conversions of the C-ABI, using the same inline
// round-to-nearest-even routines as the C++ header engine/half.hpp.
#include "../engine_internal.hpp"

#include <engine/half.hpp>

extern "C" {

int eng_f32_to_f16_host(const float* in, eng_half* out, std::size_t n) {
  return eng::guarded([&] {
    if (n == 0) return;
    ENG_CHECK(in != nullptr && out != nullptr, "eng_f32_to_f16_host: null pointer");
    for (std::size_t i = 0; i < n; ++i) out[i] = engine::float_to_half_bits(in[i]);
  });
}

int eng_f16_to_f32_host(const eng_half* in, float* out, std::size_t n) {
  return eng::guarded([&] {
    if (n == 0) return;
    ENG_CHECK(in != nullptr && out != nullptr, "eng_f16_to_f32_host: null pointer");
    for (std::size_t i = 0; i < n; ++i) out[i] = engine::half_bits_to_float(in[i]);
  });
}

}  // extern "C"
