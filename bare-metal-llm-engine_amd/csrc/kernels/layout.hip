// layout.hip -- weight layout conversion: dst[c][r] = src[r][c].
//
// The reference stores GEMV / RMSNorm+linear weights [K x N] (out = x . W,
// include/engine/kernels.hpp:83-99); the output-major entry points of this
// library take W [N x K], the faster decode layout on MI355X. This transpose
// converts a weight matrix once, at load time (the data movement only: bit
// patterns are copied, never converted, so it is exact for any value).
//
// One 256-thread workgroup moves 64 x 64 tiles through LDS, looping over
// tiles in a grid sized to about eight workgroups per CU, with the next
// tile's loads in flight while the current one is written out. Rows of the tile
// are read with 16-byte loads (8 halves or 4 floats per lane, consecutive
// lanes along a source row) and written back with 16-byte stores along
// destination rows; the LDS tile keeps one element per 32-bit word with a
// 65-word row pitch, so the column reads of the write-back are spread over
// the banks. When a dimension is not a multiple of the 16-byte vector, or a
// pointer is not 16-byte aligned, every element is moved on its own.
#include "launch.hpp"

#include <algorithm>
#include <cstdint>
#include <type_traits>

namespace eng {
namespace {

constexpr int kTile = 64;
constexpr int kThreads = 256;

template <typename T, bool VEC>
__global__ __launch_bounds__(kThreads) void transpose_kernel(const T* __restrict__ src,
                                                             T* __restrict__ dst, long long rows,
                                                             long long cols) {
  static_assert(sizeof(T) == 2 || sizeof(T) == 4, "16- or 32-bit elements");
  constexpr int E = 16 / static_cast<int>(sizeof(T));  // elements per 16-byte chunk
  constexpr int CPR = kTile / E;                       // chunks per tile row
  constexpr int RPP = kThreads / CPR;                  // tile rows per pass
  typedef T vec_t __attribute__((ext_vector_type(E)));
  __shared__ uint32_t tile[kTile][kTile + 1];

  const int t = threadIdx.x;
  const int sub = t / CPR;  // tile row (load) / tile column (store) within a pass
  const int ch = t % CPR;   // chunk along the row
  const long long tiles_c = (cols + kTile - 1) / kTile;
  const long long ntiles = ((rows + kTile - 1) / kTile) * tiles_c;

  if constexpr (VEC) {
    // The next tile's loads are issued before this tile goes through LDS and
    // out, so each thread keeps two tiles' chunks in flight instead of waiting
    // for one round trip per tile. Addresses are clamped into the matrix so
    // every load is unconditional (rows past the edge re-read the last row,
    // chunks past it the last chunk: cols % E == 0); only in-range values are
    // written to LDS.
    constexpr int LP = kTile / RPP;  // chunk loads per thread per tile
    auto fetch = [&](long long tl, vec_t* v) __attribute__((always_inline)) {
      const long long r0 = tl / tiles_c * kTile;
      const long long c0 = tl % tiles_c * kTile;
      const long long gc = std::min(c0 + ch * E, cols - E);
#pragma unroll
      for (int p = 0; p < LP; ++p) {
        const long long gr = std::min(r0 + p * RPP + sub, rows - 1);
        v[p] = *reinterpret_cast<const vec_t*>(src + gr * cols + gc);
      }
    };
    vec_t cur[LP], nxt[LP];
    long long tl = blockIdx.x;
    if (tl < ntiles) fetch(tl, cur);
    for (; tl < ntiles; tl += gridDim.x) {
      const long long tn = tl + gridDim.x;
      if (tn < ntiles) fetch(tn, nxt);
      const long long r0 = tl / tiles_c * kTile;
      const long long c0 = tl % tiles_c * kTile;
#pragma unroll
      for (int p = 0; p < LP; ++p) {
        const int r = p * RPP + sub;
        if (r0 + r < rows && c0 + ch * E < cols) {
#pragma unroll
          for (int e = 0; e < E; ++e) tile[r][ch * E + e] = static_cast<uint32_t>(cur[p][e]);
        }
      }
      __syncthreads();
#pragma unroll
      for (int p = 0; p < LP; ++p) {
        const int c = p * RPP + sub;        // source column = destination row
        const long long gdr = c0 + c;
        const long long gdc = r0 + ch * E;  // destination column = source row
        if (gdr < cols && gdc < rows) {     // rows % E == 0
          vec_t v;
#pragma unroll
          for (int e = 0; e < E; ++e) v[e] = static_cast<T>(tile[ch * E + e][c]);
          *reinterpret_cast<vec_t*>(dst + gdr * rows + gdc) = v;
        }
      }
      __syncthreads();
#pragma unroll
      for (int p = 0; p < LP; ++p) cur[p] = nxt[p];
    }
  } else {
    for (long long tl = blockIdx.x; tl < ntiles; tl += gridDim.x) {
      const long long r0 = tl / tiles_c * kTile;
      const long long c0 = tl % tiles_c * kTile;
#pragma unroll
      for (int p = 0; p < kTile / RPP; ++p) {
        const int r = p * RPP + sub;
        const long long gr = r0 + r;
        const long long gc = c0 + ch * E;
#pragma unroll
        for (int e = 0; e < E; ++e) {
          if (gr < rows && gc + e < cols) tile[r][ch * E + e] = static_cast<uint32_t>(src[gr * cols + gc + e]);
        }
      }
      __syncthreads();
#pragma unroll
      for (int p = 0; p < kTile / RPP; ++p) {
        const int c = p * RPP + sub;
        const long long gdr = c0 + c;
        const long long gdc = r0 + ch * E;
#pragma unroll
        for (int e = 0; e < E; ++e) {
          if (gdr < cols && gdc + e < rows) dst[gdr * rows + gdc + e] = static_cast<T>(tile[ch * E + e][c]);
        }
      }
      __syncthreads();
    }
  }
}

template <typename T>
void launch_transpose(const void* src, void* dst, long long rows, long long cols, hipStream_t s) {
  constexpr int E = 16 / static_cast<int>(sizeof(T));
  const long long ntiles = ((rows + kTile - 1) / kTile) * ((cols + kTile - 1) / kTile);
  const unsigned grid =
      static_cast<unsigned>(std::max(1LL, std::min(ntiles, 8LL * device_cu_count())));
  const bool vec = rows % E == 0 && cols % E == 0 && aligned_to(src, 16) && aligned_to(dst, 16);
  if (vec) {
    transpose_kernel<T, true><<<grid, kThreads, 0, s>>>(static_cast<const T*>(src),
                                                        static_cast<T*>(dst), rows, cols);
  } else {
    transpose_kernel<T, false><<<grid, kThreads, 0, s>>>(static_cast<const T*>(src),
                                                         static_cast<T*>(dst), rows, cols);
  }
  ENG_LAUNCH_CHECK();
}

void check_transpose(const void* src, const void* dst, int64_t rows, int64_t cols,
                     std::size_t esize) {
  ENG_CHECK(rows >= 0 && cols >= 0, "transpose: negative dimension");
  if (rows == 0 || cols == 0) return;
  ENG_CHECK(src != nullptr && dst != nullptr, "transpose: null device pointer");
  const auto a = reinterpret_cast<std::uintptr_t>(src);
  const auto b = reinterpret_cast<std::uintptr_t>(dst);
  const auto bytes = static_cast<std::uintptr_t>(rows) * static_cast<std::uintptr_t>(cols) * esize;
  ENG_CHECK(a + bytes <= b || b + bytes <= a, "transpose: src and dst overlap (in-place is not supported)");
}

}  // namespace
}  // namespace eng

using eng::guarded;

extern "C" {

int eng_transpose_f16(const eng_half* src, eng_half* dst, int64_t rows, int64_t cols,
                      eng_stream stream) {
  return guarded([&] {
    eng::check_transpose(src, dst, rows, cols, 2);
    if (rows == 0 || cols == 0) return;
    eng::launch_transpose<uint16_t>(src, dst, rows, cols, eng::as_stream(stream));
  });
}

int eng_transpose_f32(const float* src, float* dst, int64_t rows, int64_t cols,
                      eng_stream stream) {
  return guarded([&] {
    eng::check_transpose(src, dst, rows, cols, 4);
    if (rows == 0 || cols == 0) return;
    eng::launch_transpose<uint32_t>(src, dst, rows, cols, eng::as_stream(stream));
  });
}

}  // extern "C"
