#pragma once
//===----------------------------------------------------------------------===//
// engine/hip_device.hpp -- device discovery and reporting on HIP.
//
// HIP counterpart of the reference's include/engine/cuda_device.hpp:20-48,
// served by the C-ABI (eng_device_* in engine_hip.h). Like the reference, the
// count is 0 rather than an error when no device or driver is present, and the
// summary is safe to call unconditionally.
//===----------------------------------------------------------------------===//

#include <engine/check.hpp>

#include <cstdio>
#include <string>

namespace engine {

inline int hip_device_count() {
  int n = 0;
  return eng_device_count(&n) == ENG_OK ? n : 0;
}

/// e.g. "AMD Instinct MI355X | gfx950:sramecc+:xnack- | 288.0 GiB | 256 CUs | 160 KiB LDS/block | 8000.0 GB/s"
inline std::string hip_device_summary() {
  char buf[512];
  ENGINE_ABI_CHECK(eng_device_summary(buf, sizeof(buf)));
  return buf;
}

/// Peak HBM bandwidth in GB/s (the published figure for known parts).
inline double hip_peak_bandwidth_gbs() {
  double v = 0.0;
  ENGINE_ABI_CHECK(eng_peak_bandwidth_gbs(&v));
  return v;
}

inline std::string hip_driver_version() {
  char buf[64];
  ENGINE_ABI_CHECK(eng_driver_version(buf, sizeof(buf)));
  return buf;
}

inline int hip_clock_rate_khz() {
  int v = 0;
  ENGINE_ABI_CHECK(eng_clock_rate_khz(&v));
  return v;
}

inline int hip_live_sm_clock_mhz() {
  int v = 0;
  ENGINE_ABI_CHECK(eng_live_sm_clock_mhz(&v));
  return v;
}

inline int hip_live_mem_clock_mhz() {
  int v = 0;
  ENGINE_ABI_CHECK(eng_live_mem_clock_mhz(&v));
  return v;
}

inline std::string hip_device_arch() {
  char buf[128];
  ENGINE_ABI_CHECK(eng_device_arch(buf, sizeof(buf)));
  return buf;
}

/// Prints the summary and warns when the device is not the build's target.
inline void print_hip_device_info() {
  if (hip_device_count() == 0) {
    std::printf("HIP: no device is visible.\n");
    return;
  }
  const std::string arch = hip_device_arch();
  std::printf("HIP device: %s\n", hip_device_summary().c_str());
  std::printf("  driver %s, clock %d MHz, memory clock %d MHz, built for %s\n",
              hip_driver_version().c_str(), hip_clock_rate_khz() / 1000,
              hip_live_mem_clock_mhz(), ENGINE_HIP_ARCH_STRING);
  if (arch.compare(0, 6, ENGINE_HIP_ARCH_STRING) != 0) {
    std::printf("  WARNING: this library was built for %s but the device is %s.\n",
                ENGINE_HIP_ARCH_STRING, arch.c_str());
  }
}

}  // namespace engine
