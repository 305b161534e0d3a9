#pragma once
//===----------------------------------------------------------------------===//
// engine/config.hpp -- build configuration of the MI355X engine.
//
// Counterpart of the reference's CMake-generated engine/config.hpp
// (reference cmake/engine_config.hpp.in:8-21). This build has one target, so
// the file is static: HIP is always present and the device code is gfx950.
//===----------------------------------------------------------------------===//

#define ENGINE_HAS_HIP 1
#define ENGINE_HIP_ARCH_STRING "gfx950"
#define ENGINE_VERSION_STRING "0.2"
