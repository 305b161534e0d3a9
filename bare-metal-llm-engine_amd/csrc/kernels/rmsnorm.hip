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

// Sum over the workgroup (four waves), returned to every thread; red holds
// four floats and is free again when this returns.
__device__ __forceinline__ float block_sum(float v, float* red) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  const float total = red[0] + red[1] + red[2] + red[3];
  __syncthreads();
  return total;
}

__device__ __forceinline__ float block_max(float v, float* red) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off));
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  const float m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  __syncthreads();
  return m;
}

// RMSNorm rows for the fp16 matrix cores: v = in * s_r * weight exactly as
// rmsnorm_kernel<true> computes it (same per-thread order, same reduction),
// scaled by 2^e_r so the row's largest |v| lies in [2^14, 2^15), and written
// as three fp16 planes h1 = fp16(a), h2 = fp16(a - h1), h3 = fp16(a - h1 -
// h2) of a = v 2^e_r; rscale[r] = 2^-e_r. Three 11-bit terms hold all 24
// bits of a while |a| >= 2^-14 (fp16's smallest normal); smaller values err
// by at most 2^-25, 2^-39 of the row's largest. An all-zero or non-finite row
// keeps e_r = 0. Planes are K-blocked: value (r, c) of plane p sits at
// planes[p rows cols + ((c / 32) rows + r) 32 + c % 32], so the 32-column
// block of any run of rows is one contiguous slab (a 128-row GEMM tile of one
// K step is 8 KiB in one piece). Needs cols % 32 == 0 and 16-byte aligned in.
// One workgroup per row (grid-stride); the row's first KPER float4 per thread
// and their gamma values are loaded together up front and stay in registers
// between the three passes (gamma loaded only in the second pass cost a
// second memory round trip behind the first reduction); the rest is read
// again.
template <int KPER>
__global__ __launch_bounds__(kThreads) void rmsnorm_split3_kernel(
    const float* __restrict__ in, const float* __restrict__ weight, _Float16* __restrict__ planes,
    float* __restrict__ rscale, long long rows, long long cols, float eps) {
  typedef _Float16 half4 __attribute__((ext_vector_type(4)));
  __shared__ float red[kThreads / 64];
  const int t = threadIdx.x;
  const long long plane = rows * cols;
  const long long n4 = cols / 4;
  for (long long r = blockIdx.x; r < rows; r += gridDim.x) {
    const float4* src = reinterpret_cast<const float4*>(in + r * cols);
    const float* wp = weight != nullptr ? weight : in;  // read and unused when null
    float4 keep[KPER];
    float4 wk[KPER];
#pragma unroll
    for (int j = 0; j < KPER; ++j) {
      const long long i = t + static_cast<long long>(j) * kThreads;
      const long long ic = i < n4 ? i : 0;
      keep[j] = src[ic];
      wk[j] = make_float4(wp[4 * ic], wp[4 * ic + 1], wp[4 * ic + 2], wp[4 * ic + 3]);
    }
    float ss = 0.0f;
    auto add_sq = [&](float4 v) {
      ss = fmaf(v.x, v.x, ss);
      ss = fmaf(v.y, v.y, ss);
      ss = fmaf(v.z, v.z, ss);
      ss = fmaf(v.w, v.w, ss);
    };
#pragma unroll
    for (int j = 0; j < KPER; ++j)
      if (t + static_cast<long long>(j) * kThreads < n4) add_sq(keep[j]);
    for (long long i = t + static_cast<long long>(KPER) * kThreads; i < n4; i += kThreads)
      add_sq(src[i]);
    const float scale = 1.0f / sqrtf(block_sum(ss, red) / static_cast<float>(cols) + eps);
    auto value = [&](float4 v, float4 gw) {
      v.x *= scale;
      v.y *= scale;
      v.z *= scale;
      v.w *= scale;
      if (weight != nullptr) {
        v.x *= gw.x;
        v.y *= gw.y;
        v.z *= gw.z;
        v.w *= gw.w;
      }
      return v;
    };
    auto gamma_at = [&](long long i) {
      return weight != nullptr ? make_float4(weight[4 * i], weight[4 * i + 1], weight[4 * i + 2],
                                             weight[4 * i + 3])
                               : make_float4(1.0f, 1.0f, 1.0f, 1.0f);
    };
    auto amax = [](float m, float4 v) {
      return fmaxf(fmaxf(fmaxf(m, fabsf(v.x)), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
    };
    float mx = 0.0f;
#pragma unroll
    for (int j = 0; j < KPER; ++j) {
      const long long i = t + static_cast<long long>(j) * kThreads;
      if (i < n4) {
        keep[j] = value(keep[j], wk[j]);
        mx = amax(mx, keep[j]);
      }
    }
    for (long long i = t + static_cast<long long>(KPER) * kThreads; i < n4; i += kThreads)
      mx = amax(mx, value(src[i], gamma_at(i)));
    mx = block_max(mx, red);
    int e = 0;
    if (mx > 0.0f && mx <= 3.4028235e38f) {
      int ex = 0;
      frexpf(mx, &ex);  // mx in [2^(ex - 1), 2^ex)
      e = min(15 - ex, 126);
    }
    auto put = [&](long long i, float4 v) {
      const long long c = 4 * i;
      _Float16* dst = planes + ((c >> 5) * rows + r) * 32 + (c & 31);
      const float a[4] = {ldexpf(v.x, e), ldexpf(v.y, e), ldexpf(v.z, e), ldexpf(v.w, e)};
      half4 h1, h2, h3;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        h1[q] = static_cast<_Float16>(a[q]);
        const float r1 = a[q] - static_cast<float>(h1[q]);
        h2[q] = static_cast<_Float16>(r1);
        h3[q] = static_cast<_Float16>(r1 - static_cast<float>(h2[q]));
      }
      *reinterpret_cast<half4*>(dst) = h1;
      *reinterpret_cast<half4*>(dst + plane) = h2;
      *reinterpret_cast<half4*>(dst + 2 * plane) = h3;
    };
#pragma unroll
    for (int j = 0; j < KPER; ++j) {
      const long long i = t + static_cast<long long>(j) * kThreads;
      if (i < n4) put(i, keep[j]);
    }
    for (long long i = t + static_cast<long long>(KPER) * kThreads; i < n4; i += kThreads)
      put(i, value(src[i], gamma_at(i)));
    if (t == 0) rscale[r] = ldexpf(1.0f, -e);
  }
}

}  // namespace

void launch_rmsnorm_split3(const float* in, const float* weight, _Float16* planes, float* rscale,
                           long long rows, long long cols, float eps, hipStream_t stream) {
  ENG_CHECK(cols % 32 == 0 && aligned_to(in, 16) && aligned_to(planes, 16),
            "rmsnorm split: needs cols % 32 == 0 and 16-byte aligned rows");
  const long long wanted = 32LL * device_cu_count();
  const unsigned grid = static_cast<unsigned>(std::min(rows, wanted));
  if (cols <= 4LL * 4 * kThreads) {
    rmsnorm_split3_kernel<4><<<grid, kThreads, 0, stream>>>(in, weight, planes, rscale, rows, cols,
                                                             eps);
  } else {
    rmsnorm_split3_kernel<8><<<grid, kThreads, 0, stream>>>(in, weight, planes, rscale, rows, cols,
                                                             eps);
  }
  ENG_LAUNCH_CHECK();
}

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
