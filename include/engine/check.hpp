#pragma once
//===----------------------------------------------------------------------===//
// engine/check.hpp -- error contract of the engine's C++ API.
//
// Same contract as the reference (include/engine/check.hpp:36-107):
//   * engine::EngineError (a std::runtime_error) for every failure, with the
//     message "[engine] <file>:<line>\n  check failed: <expr>\n  <message>";
//   * ENGINE_CHECK: always-on precondition; ENGINE_ASSERT: debug-only;
//   * HIP_CHECK wraps HIP runtime calls made by user code; HIP_CHECK_KERNEL,
//     placed after a kernel launch, reports launch errors and -- in debug
//     builds or with ENGINE_ALWAYS_SYNC_CHECK -- synchronises so an in-kernel
//     fault is attributed to that line (CUDA_CHECK_KERNEL, :94-107);
//   * ENGINE_ABI_CHECK turns a non-zero status of the engine's C-ABI into an
//     EngineError carrying the library's own message (eng_last_error()).
//===----------------------------------------------------------------------===//

#include <engine/config.hpp>
#include <engine_hip.h>

#include <hip/hip_runtime_api.h>

#include <sstream>
#include <stdexcept>
#include <string>

namespace engine {

class EngineError : public std::runtime_error {
 public:
  explicit EngineError(const std::string& what) : std::runtime_error(what) {}
};

namespace detail {

[[noreturn]] inline void throw_error(const char* file, int line, const char* expr,
                                     const std::string& msg) {
  std::ostringstream oss;
  oss << "[engine] " << file << ":" << line << "\n"
      << "  check failed: " << expr << "\n"
      << "  " << msg;
  throw EngineError(oss.str());
}

inline void check_hip(hipError_t err, const char* file, int line, const char* expr) {
  if (err != hipSuccess) {
    std::ostringstream oss;
    oss << hipGetErrorName(err) << ": " << hipGetErrorString(err);
    throw_error(file, line, expr, oss.str());
  }
}

inline void check_status(int status) {
  if (status != ENG_OK) throw EngineError(eng_last_error());
}

}  // namespace detail
}  // namespace engine

#define ENGINE_CHECK(cond, msg)                                        \
  do {                                                                 \
    if (!(cond)) {                                                     \
      ::engine::detail::throw_error(__FILE__, __LINE__, #cond, (msg)); \
    }                                                                  \
  } while (0)

#ifdef NDEBUG
#define ENGINE_ASSERT(cond, msg) ((void)0)
#else
#define ENGINE_ASSERT(cond, msg) ENGINE_CHECK(cond, msg)
#endif

#define HIP_CHECK(call) ::engine::detail::check_hip((call), __FILE__, __LINE__, #call)

// After a kernel launch in user code: the launch-configuration error always;
// in debug builds (or with ENGINE_ALWAYS_SYNC_CHECK) also a device
// synchronisation, so execution faults surface at this line.
#if !defined(NDEBUG) || defined(ENGINE_ALWAYS_SYNC_CHECK)
#define HIP_CHECK_KERNEL()                  \
  do {                                      \
    HIP_CHECK(hipGetLastError());           \
    HIP_CHECK(hipDeviceSynchronize());      \
  } while (0)
#else
#define HIP_CHECK_KERNEL() HIP_CHECK(hipGetLastError())
#endif

#define ENGINE_ABI_CHECK(call) ::engine::detail::check_status(call)
