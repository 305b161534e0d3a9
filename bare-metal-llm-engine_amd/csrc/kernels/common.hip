// common.hip -- zero-fill kernel and the per-stream split-K GEMV workspace.
#include "../engine_internal.hpp"

#include <map>
#include <mutex>
#include <utility>

namespace eng {
namespace {

// Grid-stride zero fill; 16-byte stores for the aligned body, bytes for the rest.
__global__ __launch_bounds__(256) void fill_zero_kernel(unsigned char* __restrict__ p,
                                                        std::size_t bytes) {
  const std::size_t tid = static_cast<std::size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const std::size_t stride = static_cast<std::size_t>(gridDim.x) * blockDim.x;
  const std::size_t head = (16 - (reinterpret_cast<std::uintptr_t>(p) & 15)) & 15;
  const std::size_t pre = head < bytes ? head : bytes;
  for (std::size_t i = tid; i < pre; i += stride) p[i] = 0;
  uint4* body = reinterpret_cast<uint4*>(p + pre);
  const std::size_t nvec = (bytes - pre) / 16;
  for (std::size_t i = tid; i < nvec; i += stride) body[i] = make_uint4(0, 0, 0, 0);
  for (std::size_t i = pre + nvec * 16 + tid; i < bytes; i += stride) p[i] = 0;
}

// Workspace sizes: 4 MiB of fp32 partials bounds nsplit * N.
constexpr std::size_t kPartials = std::size_t{1} << 20;
constexpr std::size_t kPartialSs = std::size_t{1} << 12;

struct Key {
  int device;
  hipStream_t stream;
  bool operator<(const Key& o) const {
    return device != o.device ? device < o.device : stream < o.stream;
  }
};

std::mutex g_ws_mu;
std::map<Key, GemvWorkspace>& workspaces() {
  static auto* m = new std::map<Key, GemvWorkspace>();  // leaked: no exit-time teardown
  return *m;
}

}  // namespace

void fill_zero_async(void* ptr, std::size_t bytes, hipStream_t stream) {
  if (bytes == 0) return;
  const std::size_t vec = bytes / 16 + 1;
  std::size_t blocks = (vec + 255) / 256;
  if (blocks > 4096) blocks = 4096;
  fill_zero_kernel<<<static_cast<unsigned>(blocks), 256, 0, stream>>>(
      static_cast<unsigned char*>(ptr), bytes);
  ENG_LAUNCH_CHECK();
}

GemvWorkspace& gemv_workspace(hipStream_t stream) {
  int dev = 0;
  ENG_HIP_CHECK(hipGetDevice(&dev));
  std::lock_guard<std::mutex> lock(g_ws_mu);
  auto& m = workspaces();
  auto it = m.find(Key{dev, stream});
  if (it != m.end()) return it->second;

  GemvWorkspace ws;
  ws.capacity_partials = kPartials;
  ws.capacity_ss = kPartialSs;
  void* base = nullptr;
  ENG_HIP_CHECK(hipMalloc(&base, (kPartials + kPartialSs) * sizeof(float)));
  ws.partials = static_cast<float*>(base);
  ws.partial_ss = ws.partials + kPartials;
  return m.emplace(Key{dev, stream}, ws).first->second;
}

void release_gemv_workspace(hipStream_t stream) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) {
    (void)hipGetLastError();
    return;
  }
  std::lock_guard<std::mutex> lock(g_ws_mu);
  auto& m = workspaces();
  auto it = m.find(Key{dev, stream});
  if (it == m.end()) return;
  (void)hipFree(it->second.partials);
  m.erase(it);
}

}  // namespace eng
