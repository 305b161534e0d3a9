// common.hip -- fill and delay kernels and the per-stream scratch arenas.
#include "../engine_internal.hpp"

#include <algorithm>
#include <map>
#include <memory>
#include <mutex>
#include <utility>
#include <vector>

namespace eng {
namespace {

// Grid-stride byte fill; 16-byte stores for the aligned body, bytes for the rest.
__global__ __launch_bounds__(256) void fill_bytes_kernel(unsigned char* __restrict__ p,
                                                         std::size_t bytes, unsigned value) {
  const std::size_t tid = static_cast<std::size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const std::size_t stride = static_cast<std::size_t>(gridDim.x) * blockDim.x;
  const std::size_t head = (16 - (reinterpret_cast<std::uintptr_t>(p) & 15)) & 15;
  const std::size_t pre = head < bytes ? head : bytes;
  const unsigned char b = static_cast<unsigned char>(value);
  const unsigned word = b * 0x01010101u;
  for (std::size_t i = tid; i < pre; i += stride) p[i] = b;
  uint4* body = reinterpret_cast<uint4*>(p + pre);
  const std::size_t nvec = (bytes - pre) / 16;
  for (std::size_t i = tid; i < nvec; i += stride) body[i] = make_uint4(word, word, word, word);
  for (std::size_t i = pre + nvec * 16 + tid; i < bytes; i += stride) p[i] = b;
}

// One wave that sleeps until `ticks` of the constant-rate wall clock have
// passed since it started; every lane leaves once the deadline is reached, so
// the wait is bounded by its argument.
__global__ __launch_bounds__(64) void stream_delay_kernel(unsigned long long ticks) {
  const unsigned long long start = wall_clock64();
  while (wall_clock64() - start < ticks) __builtin_amdgcn_s_sleep(127);
}

struct Key {
  int device;
  hipStream_t stream;
  int level;
  bool operator<(const Key& o) const {
    if (device != o.device) return device < o.device;
    if (stream != o.stream) return stream < o.stream;
    return level < o.level;
  }
};

constexpr int kScratchLevels = 3;

struct Arena {
  std::mutex mu;  // held by the live lease
  void* base = nullptr;
  std::size_t capacity = 0;
  std::vector<void*> retired;  // outgrown blocks, kept for kernels still queued on them
  bool captured = false;       // leased while the stream was capturing
};

constexpr std::size_t kMinArena = std::size_t{1} << 20;

std::mutex g_arenas_mu;  // guards the map, not the arenas
std::map<Key, std::unique_ptr<Arena>>& arenas() {
  static auto* m = new std::map<Key, std::unique_ptr<Arena>>();  // leaked: no exit-time teardown
  return *m;
}

}  // namespace

void fill_bytes_async(void* ptr, int value, std::size_t bytes, hipStream_t stream) {
  if (bytes == 0) return;
  const std::size_t vec = bytes / 16 + 1;
  std::size_t blocks = (vec + 255) / 256;
  if (blocks > 4096) blocks = 4096;
  fill_bytes_kernel<<<static_cast<unsigned>(blocks), 256, 0, stream>>>(
      static_cast<unsigned char*>(ptr), bytes, static_cast<unsigned>(value) & 0xFFu);
  ENG_LAUNCH_CHECK();
}

void fill_zero_async(void* ptr, std::size_t bytes, hipStream_t stream) {
  fill_bytes_async(ptr, 0, bytes, stream);
}

void stream_delay_async(unsigned microseconds, hipStream_t stream) {
  if (microseconds == 0) return;
  int dev = 0, khz = 0;
  ENG_HIP_CHECK(hipGetDevice(&dev));
  ENG_HIP_CHECK(hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, dev));
  ENG_CHECK(khz > 0, "eng_stream_delay: the device reports no constant clock rate");
  const unsigned long long ticks = static_cast<unsigned long long>(khz) * microseconds / 1000ull;
  stream_delay_kernel<<<1, 64, 0, stream>>>(ticks);
  ENG_LAUNCH_CHECK();
}

StreamScratch::StreamScratch(hipStream_t stream, std::size_t bytes, int level) {
  ENG_CHECK(level >= 0 && level < kScratchLevels, "stream scratch: no such level");
  int dev = 0;
  ENG_HIP_CHECK(hipGetDevice(&dev));
  Arena* arena = nullptr;
  {
    std::lock_guard<std::mutex> lock(g_arenas_mu);
    auto& slot = arenas()[Key{dev, stream, level}];
    if (!slot) slot = std::make_unique<Arena>();
    arena = slot.get();
  }
  std::unique_lock<std::mutex> lock(arena->mu);
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  const hipError_t query = hipStreamIsCapturing(stream, &cap);
  if (query != hipSuccess) {
    (void)hipGetLastError();  // not left for the next launch check to report
    cap = hipStreamCaptureStatusNone;
  }
  if (cap != hipStreamCaptureStatusNone) arena->captured = true;
  if (bytes > arena->capacity) {
    // Growing allocates, which a stream under HIP graph capture may not do:
    // the capture needs an arena already sized by the same work run eagerly.
    ENG_HIP_CHECK(query);
    ENG_CHECK(cap == hipStreamCaptureStatusNone,
              "stream scratch: this call needs a larger scratch arena than the capturing "
              "stream has; run the same work once eagerly on this stream before capturing it");
    // The outgrown block stays allocated until the stream's arenas are
    // released: queued kernels still address it. (Doubling keeps the retired
    // blocks below the current one's size in total.)
    const std::size_t want = std::max({bytes, kMinArena, 2 * arena->capacity});
    void* grown = nullptr;
    ENG_HIP_CHECK(hipMalloc(&grown, want));
    if (arena->base != nullptr) arena->retired.push_back(arena->base);
    arena->base = grown;
    arena->capacity = want;
  }
  ptr_ = arena->base;
  held_ = lock.release();
}

StreamScratch::~StreamScratch() {
  if (held_ != nullptr) held_->unlock();
}

namespace {
// The arena of (current device, stream, level), or nullptr.
Arena* find_arena(hipStream_t stream, int level) {
  int dev = 0;
  ENG_HIP_CHECK(hipGetDevice(&dev));
  std::lock_guard<std::mutex> lock(g_arenas_mu);
  auto& m = arenas();
  auto it = m.find(Key{dev, stream, level});
  return it == m.end() ? nullptr : it->second.get();
}
}  // namespace

void begin_capture_scratch(hipStream_t stream) {
  for (int level = 0; level < kScratchLevels; ++level) {
    Arena* arena = find_arena(stream, level);
    if (arena == nullptr) continue;
    std::lock_guard<std::mutex> lock(arena->mu);
    arena->captured = false;
  }
}

void adopt_stream_scratch(hipStream_t stream, std::vector<void*>& owned) {
  for (int level = 0; level < kScratchLevels; ++level) {
    Arena* arena = find_arena(stream, level);
    if (arena == nullptr) continue;
    std::lock_guard<std::mutex> lock(arena->mu);
    if (!arena->captured || arena->base == nullptr) continue;
    // Fresh block first: if it cannot be allocated, the arena is unchanged.
    // (Growth is refused during capture, so the captured kernels address
    // only the current block; outgrown blocks stay with the arena.)
    void* fresh = nullptr;
    ENG_HIP_CHECK(hipMalloc(&fresh, arena->capacity));
    owned.push_back(arena->base);
    arena->base = fresh;
    arena->captured = false;
  }
}

void release_stream_scratch(hipStream_t stream) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) {
    (void)hipGetLastError();
    return;
  }
  for (int level = 0; level < kScratchLevels; ++level) {
    std::unique_ptr<Arena> arena;
    {
      std::lock_guard<std::mutex> lock(g_arenas_mu);
      auto& m = arenas();
      auto it = m.find(Key{dev, stream, level});
      if (it == m.end()) continue;
      arena = std::move(it->second);
      m.erase(it);
    }
    std::lock_guard<std::mutex> lock(arena->mu);  // no lease may be live
    if (arena->base != nullptr) (void)hipFree(arena->base);
    for (void* p : arena->retired) (void)hipFree(p);
  }
}

}  // namespace eng
