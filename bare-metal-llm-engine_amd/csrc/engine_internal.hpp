// engine_internal.hpp -- shared by every translation unit of libengine_hip.so.
//
// Errors inside the library are C++ exceptions (eng::Error) carrying an ABI
// status code; every extern "C" entry point runs its body through
// eng::guarded(), which turns an exception into that status code plus the
// thread-local message returned by eng_last_error(). Message layout and the
// "always-on precondition" semantics follow the reference's check layer
// (reference include/engine/check.hpp:36-107).
#pragma once

#include <hip/hip_runtime.h>

#include <engine_hip.h>

#include <cstddef>
#include <cstdint>
#include <mutex>
#include <stdexcept>
#include <string>
#include <vector>

namespace eng {

class Error : public std::runtime_error {
 public:
  Error(int code, const std::string& what) : std::runtime_error(what), code_(code) {}
  int code() const { return code_; }

 private:
  int code_;
};

[[noreturn]] void raise(int code, const char* file, int line, const char* expr,
                        const std::string& msg);
[[noreturn]] void raise_hip(hipError_t err, const char* file, int line, const char* expr);
void set_last_error(const std::string& msg);
void clear_last_error();

// Runs `body`; returns ENG_OK or the status of the exception it threw.
template <class F>
int guarded(F&& body) noexcept {
  try {
    body();
    return ENG_OK;
  } catch (const Error& e) {
    set_last_error(e.what());
    return e.code();
  } catch (const std::bad_alloc&) {
    set_last_error("[engine] host allocation failed (std::bad_alloc)");
    return ENG_DEVICE_ERROR;
  } catch (const std::exception& e) {
    set_last_error(std::string("[engine] unexpected exception: ") + e.what());
    return ENG_DEVICE_ERROR;
  } catch (...) {
    set_last_error("[engine] unknown exception");
    return ENG_DEVICE_ERROR;
  }
}

inline hipStream_t as_stream(eng_stream s) { return reinterpret_cast<hipStream_t>(s); }
inline hipEvent_t as_event(eng_event e) { return reinterpret_cast<hipEvent_t>(e); }

inline bool aligned_to(const void* p, std::uintptr_t bytes) {
  return (reinterpret_cast<std::uintptr_t>(p) % bytes) == 0;
}

// Zero-fills `bytes` of device memory with a kernel on `stream` (used for the
// K == 0 results; a fill kernel rather than hipMemsetAsync so that callers may
// capture these launches in a HIP graph).
void fill_zero_async(void* ptr, std::size_t bytes, hipStream_t stream);
// The same fill with the low byte of `value` (eng_memset_async).
void fill_bytes_async(void* ptr, int value, std::size_t bytes, hipStream_t stream);
// A one-wave kernel on `stream` that returns after `microseconds` of GPU time
// (eng_stream_delay).
void stream_delay_async(unsigned microseconds, hipStream_t stream);

// Per-(device, stream) scratch arena for launchers whose kernels pass data to
// a later kernel of the same call (split-K GEMV and split-KV attention
// partials, the normalised rows of rmsnorm_linear at M > 1, the FFN's gate /
// up vectors). Launches on one stream run in order, so a call can reuse the
// arena as soon as the previous call's launches are queued: no event, no
// allocation per call. The lease holds the arena's lock until it goes out of
// scope, so two host threads that share a stream cannot interleave their
// kernel pairs on it; take it before the first launch that writes the arena
// and keep it past the last one that reads it. The arena grows to the largest
// request (a new block; the outgrown one stays allocated for queued kernels
// and HIP graphs captured on it) and its blocks are freed when the stream is
// destroyed through eng_stream_destroy, or at exit. A graph captured on the
// stream takes its blocks over at the end of the capture (adopt_stream_scratch)
// and the stream continues on fresh blocks, so a replay never shares scratch
// with eager calls or with another graph. Growing is refused while the stream
// is capturing (allocation is not capturable). Each
// (device, stream) has one arena per level: a launcher takes at most one lease
// per level, and a composite launcher that keeps a lease while it calls other
// launchers (the FFN's gate / up buffers around the GEMV launches, which may
// lease split-K partials) takes level 1, so the inner lease (level 0) never
// waits on its own caller's lock. The GEMM's stream-K records take level 2:
// its callers (rmsnorm_linear's normalised rows at level 0, the FFN's
// buffers at level 1) hold their leases across it.
class StreamScratch {
 public:
  StreamScratch(hipStream_t stream, std::size_t bytes, int level = 0);
  ~StreamScratch();
  StreamScratch(const StreamScratch&) = delete;
  StreamScratch& operator=(const StreamScratch&) = delete;
  void* get() const { return ptr_; }

 private:
  std::mutex* held_ = nullptr;
  void* ptr_ = nullptr;
};
void release_stream_scratch(hipStream_t stream);
// Clears the "leased during capture" mark of `stream`'s arenas (at capture begin).
void begin_capture_scratch(hipStream_t stream);
// Moves the current block of each of `stream`'s arenas that a launch leased
// while the stream was capturing into `owned`, and gives each such arena a
// fresh block of its current size. The caller (a captured graph) frees the
// moved blocks; it must first wait for the stream's eager work queued before
// the capture, which may still address them.
void adopt_stream_scratch(hipStream_t stream, std::vector<void*>& owned);

}  // namespace eng

#define ENG_CHECK(cond, msg)                                                           \
  do {                                                                                 \
    if (!(cond)) ::eng::raise(ENG_INVALID_ARGUMENT, __FILE__, __LINE__, #cond, (msg)); \
  } while (0)

#define ENG_HIP_CHECK(call)                                           \
  do {                                                                \
    hipError_t eng_err_ = (call);                                     \
    if (eng_err_ != hipSuccess) ::eng::raise_hip(eng_err_, __FILE__, __LINE__, #call); \
  } while (0)

// After a kernel launch: reports launch-configuration errors. With
// ENGINE_ALWAYS_SYNC_CHECK defined it also synchronises so in-kernel faults are
// attributed to the launching line (reference include/engine/check.hpp:94-107).
#ifdef ENGINE_ALWAYS_SYNC_CHECK
#define ENG_LAUNCH_CHECK()                     \
  do {                                         \
    ENG_HIP_CHECK(hipGetLastError());          \
    ENG_HIP_CHECK(hipDeviceSynchronize());     \
  } while (0)
#else
#define ENG_LAUNCH_CHECK() ENG_HIP_CHECK(hipGetLastError())
#endif
