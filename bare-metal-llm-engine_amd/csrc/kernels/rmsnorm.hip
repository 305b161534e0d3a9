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
    if constexpr (VEC) {
      const long long n4 = cols / 4;
      for (long long i = t; i < n4; i += kThreads) {
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
      for (long long i = t; i < n4; i += kThreads) {
        float4 v = reinterpret_cast<const float4*>(src)[i];
        v.x *= scale;
        v.y *= scale;
        v.z *= scale;
        v.w *= scale;
        if (weight != nullptr) {
          v.x *= weight[4 * i];
          v.y *= weight[4 * i + 1];
          v.z *= weight[4 * i + 2];
          v.w *= weight[4 * i + 3];
        }
        reinterpret_cast<float4*>(dst)[i] = v;
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
