// rmsnorm.hip -- row-wise RMSNorm (reference kernels/rmsnorm.cu:84-192).
//
// out[r][c] = in[r][c] * (1 / sqrt(sum_c in[r][c]^2 / cols + eps)) * weight[c]
// with eps inside the square root and weight optional. One workgroup per row
// (grid-stride over rows); the sum of squares is reduced inside each wave with
// cross-lane shuffles and across the 4 waves through LDS.
#include "launch.hpp"

#include <algorithm>

namespace eng {
namespace {

constexpr int kThreads = 256;

template <bool VEC>
__global__ __launch_bounds__(kThreads) void rmsnorm_kernel(const float* __restrict__ in,
                                                           const float* __restrict__ weight,
                                                           float* __restrict__ out,
                                                           long long rows, long long cols,
                                                           float eps) {
  __shared__ float red[kThreads / 64];
  const int t = threadIdx.x;
  for (long long r = blockIdx.x; r < rows; r += gridDim.x) {
    const float* src = in + r * cols;
    float* dst = out + r * cols;
    float ss = 0.0f;
    // VEC: the first kPer float4 items of the thread (and their weights) are
    // loaded together -- in-bounds indices, no branch around a load -- and
    // kept in registers for the second pass, so a row of up to 4 kPer kThreads
    // columns costs one round trip instead of one per item and pass; the sum
    // runs over the items in the same order as the plain loop (same bits).
    constexpr int kPer = 8;
    [[maybe_unused]] float4 keep[VEC ? kPer : 1];
    [[maybe_unused]] float4 wk[VEC ? kPer : 1];
    if constexpr (VEC) {
      const long long n4 = cols / 4;
      const float* wp = weight != nullptr ? weight : src;  // read and unused when null
#pragma unroll
      for (int j = 0; j < kPer; ++j) {
        const long long i = t + static_cast<long long>(j) * kThreads;
        const long long ic = i < n4 ? i : 0;
        keep[j] = reinterpret_cast<const float4*>(src)[ic];
        wk[j] = make_float4(wp[4 * ic], wp[4 * ic + 1], wp[4 * ic + 2], wp[4 * ic + 3]);
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int j = 0; j < kPer; ++j) {
        if (t + static_cast<long long>(j) * kThreads < n4) {
          const float4 v = keep[j];
          ss = fmaf(v.x, v.x, ss);
          ss = fmaf(v.y, v.y, ss);
          ss = fmaf(v.z, v.z, ss);
          ss = fmaf(v.w, v.w, ss);
        }
      }
      for (long long i = t + static_cast<long long>(kPer) * kThreads; i < n4; i += kThreads) {
        const float4 v = reinterpret_cast<const float4*>(src)[i];
        ss = fmaf(v.x, v.x, ss);
        ss = fmaf(v.y, v.y, ss);
        ss = fmaf(v.z, v.z, ss);
        ss = fmaf(v.w, v.w, ss);
      }
    } else {
      for (long long c = t; c < cols; c += kThreads) ss = fmaf(src[c], src[c], ss);
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off);
    if ((t & 63) == 0) red[t >> 6] = ss;
    __syncthreads();
    const float total = red[0] + red[1] + red[2] + red[3];
    const float scale = 1.0f / sqrtf(total / static_cast<float>(cols) + eps);
    if constexpr (VEC) {
      const long long n4 = cols / 4;
      auto finish = [&](long long i, float4 v, float4 g) {
        v.x *= scale;
        v.y *= scale;
        v.z *= scale;
        v.w *= scale;
        if (weight != nullptr) {
          v.x *= g.x;
          v.y *= g.y;
          v.z *= g.z;
          v.w *= g.w;
        }
        reinterpret_cast<float4*>(dst)[i] = v;
      };
#pragma unroll
      for (int j = 0; j < kPer; ++j) {
        const long long i = t + static_cast<long long>(j) * kThreads;
        if (i < n4) finish(i, keep[j], wk[j]);
      }
      for (long long i = t + static_cast<long long>(kPer) * kThreads; i < n4; i += kThreads) {
        const float4 g = weight != nullptr
                             ? make_float4(weight[4 * i], weight[4 * i + 1], weight[4 * i + 2],
                                           weight[4 * i + 3])
                             : make_float4(1.0f, 1.0f, 1.0f, 1.0f);
        finish(i, reinterpret_cast<const float4*>(src)[i], g);
      }
    } else {
      for (long long c = t; c < cols; c += kThreads) {
        float v = src[c] * scale;
        if (weight != nullptr) v *= weight[c];
        dst[c] = v;
      }
    }
    __syncthreads();  // red[] is reused by the next row
  }
}

}  // namespace

void launch_rmsnorm(const float* in, const float* weight, float* out, long long rows,
                    long long cols, float eps, hipStream_t stream) {
  const bool vec = (cols % 4 == 0) && aligned_to(in, 16) && aligned_to(out, 16);
  const long long wanted = 32LL * device_cu_count();
  const unsigned grid = static_cast<unsigned>(std::min(rows, wanted));
  if (vec) {
    rmsnorm_kernel<true><<<grid, kThreads, 0, stream>>>(in, weight, out, rows, cols, eps);
  } else {
    rmsnorm_kernel<false><<<grid, kThreads, 0, stream>>>(in, weight, out, rows, cols, eps);
  }
  ENG_LAUNCH_CHECK();
}

}  // namespace eng

extern "C" {

int eng_rmsnorm_f32(const float* in, const float* weight, float* out, int64_t rows,
                    int64_t cols, float eps, eng_stream stream) {
  return eng::guarded([&] {
    ENG_CHECK(rows >= 0 && cols >= 0, "rmsnorm: negative dimension");
    ENG_CHECK(in != nullptr && out != nullptr, "rmsnorm: null device pointer");
    ENG_CHECK(eps >= 0.0f, "rmsnorm: eps must be non-negative");
    if (rows == 0 || cols == 0) return;
    eng::launch_rmsnorm(in, weight, out, rows, cols, eps, eng::as_stream(stream));
  });
}

}  // extern "C"
