// pool_allocator.cpp -- pooled and passthrough allocators of the C-ABI.
//
// Behaviour contract of the reference PoolAllocator (include/engine/
// pool_allocator.hpp:27-148, src/pool_allocator.cpp:38-271), kept because the
// reference's allocator tests pin it:
//   * requests round up to a power of two, at least 256 B; blocks are 256-B aligned;
//   * a freed block goes to its size class and is handed out again before any
//     new memory is carved;
//   * new memory is carved from the existing slabs, newest first, and only then
//     from a new slab of max(next_slab, bucket) bytes, where next_slab starts at
//     the initial size and doubles up to 64 MiB;
//   * a GPU block freed with a stream is not reused until the work queued on
//     that stream at free time has finished (an event recorded at free time);
//   * statistics are exact: bytes_in_use counts bucket bytes.
// The passthrough allocator (reference src/allocator.cpp:42-118) forwards every
// request to the driver and counts it.
#include "../engine_internal.hpp"

#include <algorithm>
#include <cstdlib>
#include <deque>
#include <map>
#include <mutex>
#include <unordered_map>
#include <vector>

struct eng_pool_s {
  struct FreeBlock {
    void* ptr = nullptr;
    hipEvent_t ready = nullptr;  // GPU blocks: completes when reuse is safe
  };
  struct Slab {
    char* base = nullptr;
    std::size_t size = 0;
    std::size_t used = 0;
  };

  int device = ENG_DEVICE_CPU;
  std::size_t initial_slab = 0;
  std::size_t next_slab = 0;
  std::mutex mu;
  eng_alloc_stats stats{};
  std::map<std::size_t, std::deque<FreeBlock>> free_lists;
  std::unordered_map<void*, std::size_t> live;  // ptr -> bucket bytes
  std::vector<hipEvent_t> spare_events;
  std::vector<Slab> slabs;
};

namespace eng {
namespace {

constexpr std::size_t kMinBlock = 256;
constexpr std::size_t kAlign = 256;
constexpr std::size_t kMaxAutoSlab = std::size_t{64} << 20;

std::size_t bucket_for(std::size_t bytes) {
  std::size_t b = kMinBlock;
  while (b < bytes) b <<= 1;
  return b;
}

void* driver_alloc(int device, std::size_t bytes) {
  void* p = nullptr;
  if (device == ENG_DEVICE_CPU) {
    const std::size_t rounded = (bytes + kAlign - 1) / kAlign * kAlign;
    p = std::aligned_alloc(kAlign, rounded);
    ENG_CHECK(p != nullptr, "PoolAllocator: host aligned_alloc failed for " +
                                std::to_string(bytes) + " bytes");
  } else {
    ENG_HIP_CHECK(hipMalloc(&p, bytes));
  }
  return p;
}

void driver_free(int device, void* p) {
  if (p == nullptr) return;
  if (device == ENG_DEVICE_CPU) {
    std::free(p);
  } else {
    (void)hipFree(p);
  }
}

void check_device_kind(int device) {
  ENG_CHECK(device == ENG_DEVICE_CPU || device == ENG_DEVICE_GPU,
            "allocator: unsupported device " + std::to_string(device));
}

void* take(eng_pool_s& pool, void* p, std::size_t bucket) {
  pool.stats.bytes_in_use += bucket;
  pool.stats.peak_bytes_in_use = std::max(pool.stats.peak_bytes_in_use, pool.stats.bytes_in_use);
  pool.stats.num_allocs += 1;
  pool.live[p] = bucket;
  return p;
}

void* pool_allocate(eng_pool_s& pool, std::size_t bytes) {
  if (bytes == 0) return nullptr;
  const std::size_t bucket = bucket_for(bytes);
  std::lock_guard<std::mutex> lock(pool.mu);

  // 1. A freed block of this size class whose stream work has drained.
  auto fl = pool.free_lists.find(bucket);
  if (fl != pool.free_lists.end()) {
    auto& queue = fl->second;
    for (auto it = queue.begin(); it != queue.end(); ++it) {
      if (it->ready != nullptr) {
        const hipError_t q = hipEventQuery(it->ready);
        if (q == hipErrorNotReady) {
          (void)hipGetLastError();
          continue;
        }
        pool.spare_events.push_back(it->ready);
        it->ready = nullptr;
        ENG_HIP_CHECK(q);
      }
      void* p = it->ptr;
      queue.erase(it);
      return take(pool, p, bucket);
    }
  }

  // 2. Carve from an existing slab, newest first.
  for (auto s = pool.slabs.rbegin(); s != pool.slabs.rend(); ++s) {
    if (s->size - s->used >= bucket) {
      void* p = s->base + s->used;
      s->used += bucket;
      return take(pool, p, bucket);
    }
  }

  // 3. A new slab from the driver.
  const std::size_t slab_bytes = std::max(pool.next_slab, bucket);
  void* base = driver_alloc(pool.device, slab_bytes);
  pool.next_slab = std::min(kMaxAutoSlab, pool.next_slab * 2);
  pool.stats.bytes_reserved += slab_bytes;
  pool.stats.num_driver_allocs += 1;
  pool.slabs.push_back({static_cast<char*>(base), slab_bytes, bucket});
  return take(pool, base, bucket);
}

void pool_deallocate(eng_pool_s& pool, void* ptr, hipStream_t stream) {
  if (ptr == nullptr) return;
  std::lock_guard<std::mutex> lock(pool.mu);
  auto it = pool.live.find(ptr);
  ENG_CHECK(it != pool.live.end(), "PoolAllocator: pointer was not allocated by this pool");
  const std::size_t bucket = it->second;

  hipEvent_t ev = nullptr;
  if (pool.device == ENG_DEVICE_GPU) {
    if (!pool.spare_events.empty()) {
      ev = pool.spare_events.back();
      pool.spare_events.pop_back();
    } else {
      ENG_HIP_CHECK(hipEventCreateWithFlags(&ev, hipEventDisableTiming));
    }
    const hipError_t err = hipEventRecord(ev, stream);
    if (err != hipSuccess) {
      pool.spare_events.push_back(ev);
      ENG_HIP_CHECK(err);
    }
  }
  pool.live.erase(it);
  pool.stats.bytes_in_use -= bucket;
  pool.free_lists[bucket].push_back({ptr, ev});
}

void pool_reset(eng_pool_s& pool) {
  std::lock_guard<std::mutex> lock(pool.mu);
  for (auto& kv : pool.free_lists) {
    for (auto& blk : kv.second) {
      if (blk.ready != nullptr) (void)hipEventDestroy(blk.ready);
    }
  }
  for (hipEvent_t ev : pool.spare_events) (void)hipEventDestroy(ev);
  pool.spare_events.clear();
  for (auto& s : pool.slabs) driver_free(pool.device, s.base);
  pool.slabs.clear();
  pool.free_lists.clear();
  pool.live.clear();
  pool.stats = eng_alloc_stats{};
  pool.next_slab = pool.initial_slab;
}

eng_pool_s* make_pool(int device, std::size_t initial) {
  auto* pool = new eng_pool_s();
  pool->device = device;
  pool->initial_slab = std::max(initial, kMinBlock);
  pool->next_slab = pool->initial_slab;
  return pool;
}

struct Passthrough {
  std::mutex mu;
  eng_alloc_stats stats{};
};

Passthrough& passthrough(int device) {
  // Leaked on purpose: no teardown ordering against the HIP runtime at exit.
  static Passthrough* cpu = new Passthrough();
  static Passthrough* gpu = new Passthrough();
  return device == ENG_DEVICE_CPU ? *cpu : *gpu;
}

}  // namespace
}  // namespace eng

using eng::guarded;

extern "C" {

int eng_pool_create(eng_pool* pool, int device, std::size_t initial_slab_bytes) {
  return guarded([&] {
    ENG_CHECK(pool != nullptr, "eng_pool_create: pool is null");
    eng::check_device_kind(device);
    *pool = eng::make_pool(device, initial_slab_bytes);
  });
}

int eng_pool_destroy(eng_pool pool) {
  return guarded([&] {
    if (pool == nullptr) return;
    eng::pool_reset(*pool);
    delete pool;
  });
}

int eng_pool_default(eng_pool* pool, int device) {
  return guarded([&] {
    ENG_CHECK(pool != nullptr, "eng_pool_default: pool is null");
    eng::check_device_kind(device);
    // Process-wide, created on first use, never destroyed (see passthrough()).
    static eng_pool_s* cpu_pool = eng::make_pool(ENG_DEVICE_CPU, std::size_t{4} << 20);
    static eng_pool_s* gpu_pool = eng::make_pool(ENG_DEVICE_GPU, std::size_t{4} << 20);
    *pool = device == ENG_DEVICE_CPU ? cpu_pool : gpu_pool;
  });
}

int eng_pool_allocate(eng_pool pool, std::size_t bytes, void** ptr) {
  return guarded([&] {
    ENG_CHECK(pool != nullptr, "eng_pool_allocate: pool is null");
    ENG_CHECK(ptr != nullptr, "eng_pool_allocate: ptr is null");
    *ptr = nullptr;
    *ptr = eng::pool_allocate(*pool, bytes);
  });
}

int eng_pool_deallocate(eng_pool pool, void* ptr, eng_stream stream) {
  return guarded([&] {
    ENG_CHECK(pool != nullptr, "eng_pool_deallocate: pool is null");
    eng::pool_deallocate(*pool, ptr, eng::as_stream(stream));
  });
}

int eng_pool_stats(eng_pool pool, eng_alloc_stats* stats) {
  return guarded([&] {
    ENG_CHECK(pool != nullptr, "eng_pool_stats: pool is null");
    ENG_CHECK(stats != nullptr, "eng_pool_stats: stats is null");
    std::lock_guard<std::mutex> lock(pool->mu);
    *stats = pool->stats;
  });
}

int eng_pool_reset(eng_pool pool) {
  return guarded([&] {
    ENG_CHECK(pool != nullptr, "eng_pool_reset: pool is null");
    eng::pool_reset(*pool);
  });
}

int eng_passthrough_allocate(int device, std::size_t bytes, void** ptr) {
  return guarded([&] {
    ENG_CHECK(ptr != nullptr, "eng_passthrough_allocate: ptr is null");
    eng::check_device_kind(device);
    *ptr = nullptr;
    if (bytes == 0) return;
    void* p = eng::driver_alloc(device, bytes);
    auto& pt = eng::passthrough(device);
    std::lock_guard<std::mutex> lock(pt.mu);
    pt.stats.bytes_in_use += bytes;
    pt.stats.bytes_reserved += bytes;
    pt.stats.peak_bytes_in_use = std::max(pt.stats.peak_bytes_in_use, pt.stats.bytes_in_use);
    pt.stats.num_allocs += 1;
    pt.stats.num_driver_allocs += 1;  // every request goes to the driver
    *ptr = p;
  });
}

int eng_passthrough_deallocate(int device, void* ptr) {
  return guarded([&] {
    eng::check_device_kind(device);
    // A bare pointer carries no size, so bytes_in_use is not decremented
    // (the reference's passthrough behaves the same way).
    eng::driver_free(device, ptr);
  });
}

int eng_passthrough_stats(int device, eng_alloc_stats* stats) {
  return guarded([&] {
    ENG_CHECK(stats != nullptr, "eng_passthrough_stats: stats is null");
    eng::check_device_kind(device);
    auto& pt = eng::passthrough(device);
    std::lock_guard<std::mutex> lock(pt.mu);
    *stats = pt.stats;
  });
}

}  // extern "C"
