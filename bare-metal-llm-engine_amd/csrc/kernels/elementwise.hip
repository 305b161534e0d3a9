// elementwise.hip -- the ops either side of the linear layers of a SwiGLU FFN:
//   vector_add        out = a + b                      (reference kernels/vector_add.cu)
//   swiglu(_fp16)     out = SiLU(gate) * up            (reference kernels/swiglu.cu)
//   residual_rmsnorm  sum = x + residual, norm = RMSNorm(sum) * weight
//                                                      (reference kernels/residual_rmsnorm.cu)
// All are HBM-bound streams. vector_add and swiglu move 16 bytes per lane per
// access (float4 / 8 halves) in a grid-stride loop sized to about 8 workgroups
// per CU, falling back to scalar accesses for unaligned pointers or ragged
// sizes. residual_rmsnorm runs one 256-thread workgroup per row: the row sum
// is written once, kept in registers for the second pass (rows up to 8192
// floats; longer rows recompute x + residual, which is bit-identical), and the
// sum of squares is reduced with wave shuffles and four LDS slots in a fixed
// order. Preconditions, messages and the zero-size rules are the reference's.
#include "gemv_kernels.hpp"
#include "launch.hpp"

#include <algorithm>
#include <type_traits>

namespace eng {
namespace {

constexpr int kThreads = 256;

using F4 = gemv::RawVec<float, 4>::type;
using H8 = gemv::RawVec<_Float16, 8>::type;

unsigned stream_grid(long long work_items) {
  const long long wanted = 8LL * device_cu_count();
  const long long needed = (work_items + kThreads - 1) / kThreads;
  return static_cast<unsigned>(std::max(1LL, std::min(needed, wanted)));
}

// ------------------------------------------------------------- vector_add
__global__ __launch_bounds__(kThreads) void add_vec4_kernel(const F4* __restrict__ a,
                                                            const F4* __restrict__ b,
                                                            F4* __restrict__ out, long long n4) {
  const long long stride = static_cast<long long>(gridDim.x) * kThreads;
  for (long long i = static_cast<long long>(blockIdx.x) * kThreads + threadIdx.x; i < n4;
       i += stride) {
    out[i] = a[i] + b[i];
  }
}

__global__ __launch_bounds__(kThreads) void add_scalar_kernel(const float* __restrict__ a,
                                                              const float* __restrict__ b,
                                                              float* __restrict__ out,
                                                              long long n) {
  const long long stride = static_cast<long long>(gridDim.x) * kThreads;
  for (long long i = static_cast<long long>(blockIdx.x) * kThreads + threadIdx.x; i < n;
       i += stride) {
    out[i] = a[i] + b[i];
  }
}

// ----------------------------------------------------------------- swiglu
__global__ __launch_bounds__(kThreads) void swiglu_vec4_kernel(const F4* __restrict__ g,
                                                               const F4* __restrict__ u,
                                                               F4* __restrict__ out,
                                                               long long n4) {
  const long long stride = static_cast<long long>(gridDim.x) * kThreads;
  for (long long i = static_cast<long long>(blockIdx.x) * kThreads + threadIdx.x; i < n4;
       i += stride) {
    const F4 gv = g[i];
    const F4 uv = u[i];
    F4 r;
#pragma unroll
    for (int e = 0; e < 4; ++e) r[e] = gemv::swiglu_f32(gv[e], uv[e]);
    out[i] = r;
  }
}

__global__ __launch_bounds__(kThreads) void swiglu_scalar_kernel(const float* __restrict__ g,
                                                                 const float* __restrict__ u,
                                                                 float* __restrict__ out,
                                                                 long long n) {
  const long long stride = static_cast<long long>(gridDim.x) * kThreads;
  for (long long i = static_cast<long long>(blockIdx.x) * kThreads + threadIdx.x; i < n;
       i += stride) {
    out[i] = gemv::swiglu_f32(g[i], u[i]);
  }
}

// Half in, half out; the arithmetic is the fp32 formula, rounded to half
// (nearest even) once at the end.
__global__ __launch_bounds__(kThreads) void swiglu_h8_kernel(const H8* __restrict__ g,
                                                             const H8* __restrict__ u,
                                                             H8* __restrict__ out, long long n8) {
  const long long stride = static_cast<long long>(gridDim.x) * kThreads;
  for (long long i = static_cast<long long>(blockIdx.x) * kThreads + threadIdx.x; i < n8;
       i += stride) {
    const H8 gv = g[i];
    const H8 uv = u[i];
    H8 r;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      r[e] = static_cast<_Float16>(
          gemv::swiglu_f32(static_cast<float>(gv[e]), static_cast<float>(uv[e])));
    }
    out[i] = r;
  }
}

__global__ __launch_bounds__(kThreads) void swiglu_h_scalar_kernel(
    const _Float16* __restrict__ g, const _Float16* __restrict__ u, _Float16* __restrict__ out,
    long long n) {
  const long long stride = static_cast<long long>(gridDim.x) * kThreads;
  for (long long i = static_cast<long long>(blockIdx.x) * kThreads + threadIdx.x; i < n;
       i += stride) {
    out[i] = static_cast<_Float16>(
        gemv::swiglu_f32(static_cast<float>(g[i]), static_cast<float>(u[i])));
  }
}

// ------------------------------------------------------- residual_rmsnorm
// One workgroup per row (grid-stride over rows). VEC: float4 accesses (cols %
// 4 == 0 and 16-byte aligned rows); PER = 16-byte (or 4-byte) items each
// thread keeps in registers between the passes.
template <bool VEC, int PER>
__global__ __launch_bounds__(kThreads) void residual_rmsnorm_kernel(
    const float* __restrict__ x, const float* __restrict__ res, const float* __restrict__ w,
    float* __restrict__ norm, float* __restrict__ sum, long long rows, long long cols,
    float eps) {
  using T = typename std::conditional<VEC, F4, float>::type;
  constexpr int W = VEC ? 4 : 1;
  __shared__ float red[kThreads / 64];
  const int t = threadIdx.x;
  const long long items = cols / W;
  for (long long r = blockIdx.x; r < rows; r += gridDim.x) {
    const T* xr = reinterpret_cast<const T*>(x + r * cols);
    const T* rr = reinterpret_cast<const T*>(res + r * cols);
    T* sr = reinterpret_cast<T*>(sum + r * cols);
    T* nr = reinterpret_cast<T*>(norm + r * cols);
    // The first PER items of x, the residual and the weight are loaded
    // together (in-bounds indices, no branch around a load) before any is
    // used, so a row of up to PER kThreads items costs one round trip instead
    // of one per item; the sums run in the same order (same bits).
    const T* wr = reinterpret_cast<const T*>(w != nullptr ? w : x);  // read, unused when null
    T xk[PER], rk[PER], wk[PER];
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      const long long i = t + static_cast<long long>(j) * kThreads;
      const long long ic = i < items ? i : 0;
      xk[j] = xr[ic];
      rk[j] = rr[ic];
      wk[j] = wr[ic];
    }
    __builtin_amdgcn_sched_barrier(0);
    T keep[PER];
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      const long long i = t + static_cast<long long>(j) * kThreads;
      if (i < items) {
        const T s = xk[j] + rk[j];
        sr[i] = s;
        keep[j] = s;
        if constexpr (VEC) {
#pragma unroll
          for (int e = 0; e < 4; ++e) ss = fmaf(s[e], s[e], ss);
        } else {
          ss = fmaf(s, s, ss);
        }
      }
    }
    for (long long i = t + static_cast<long long>(PER) * kThreads; i < items; i += kThreads) {
      const T s = xr[i] + rr[i];
      sr[i] = s;
      if constexpr (VEC) {
#pragma unroll
        for (int e = 0; e < 4; ++e) ss = fmaf(s[e], s[e], ss);
      } else {
        ss = fmaf(s, s, ss);
      }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off);
    if ((t & 63) == 0) red[t >> 6] = ss;
    __syncthreads();
    const float total = ((red[0] + red[1]) + red[2]) + red[3];
    const float scale = gemv::rms_scale(total, cols, eps);

    auto finish = [&](long long i, T s, T g) {
      T v = s * scale;
      if (w != nullptr) v *= g;
      nr[i] = v;
    };
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      const long long i = t + static_cast<long long>(j) * kThreads;
      if (i < items) finish(i, keep[j], wk[j]);
    }
    for (long long i = t + static_cast<long long>(PER) * kThreads; i < items; i += kThreads) {
      finish(i, xr[i] + rr[i], wr[i]);
    }
    __syncthreads();  // red[] is reused by the next row
  }
}

}  // namespace

void launch_swiglu_f32(const float* g, const float* u, float* out, long long n,
                       hipStream_t stream) {
  if (n % 4 == 0 && aligned_to(g, 16) && aligned_to(u, 16) && aligned_to(out, 16)) {
    swiglu_vec4_kernel<<<stream_grid(n / 4), kThreads, 0, stream>>>(
        reinterpret_cast<const F4*>(g), reinterpret_cast<const F4*>(u),
        reinterpret_cast<F4*>(out), n / 4);
  } else {
    swiglu_scalar_kernel<<<stream_grid(n), kThreads, 0, stream>>>(g, u, out, n);
  }
  ENG_LAUNCH_CHECK();
}

}  // namespace eng

using eng::guarded;

extern "C" {

int eng_vector_add_f32(const float* a, const float* b, float* out, int64_t n, eng_stream stream) {
  return guarded([&] {
    ENG_CHECK(n >= 0, "vector_add: n must be non-negative");
    if (n == 0) return;
    ENG_CHECK(a != nullptr && b != nullptr && out != nullptr, "vector_add: null device pointer");
    hipStream_t s = eng::as_stream(stream);
    if (n % 4 == 0 && eng::aligned_to(a, 16) && eng::aligned_to(b, 16) &&
        eng::aligned_to(out, 16)) {
      eng::add_vec4_kernel<<<eng::stream_grid(n / 4), eng::kThreads, 0, s>>>(
          reinterpret_cast<const eng::F4*>(a), reinterpret_cast<const eng::F4*>(b),
          reinterpret_cast<eng::F4*>(out), n / 4);
    } else {
      eng::add_scalar_kernel<<<eng::stream_grid(n), eng::kThreads, 0, s>>>(a, b, out, n);
    }
    ENG_LAUNCH_CHECK();
  });
}

int eng_swiglu_f32(const float* gate, const float* up, float* out, int64_t n, eng_stream stream) {
  return guarded([&] {
    ENG_CHECK(gate != nullptr, "swiglu: gate is null");
    ENG_CHECK(up != nullptr, "swiglu: up is null");
    ENG_CHECK(out != nullptr, "swiglu: out is null");
    ENG_CHECK(n >= 0, "swiglu: n must be non-negative");
    if (n == 0) return;
    eng::launch_swiglu_f32(gate, up, out, n, eng::as_stream(stream));
  });
}

int eng_swiglu_f16(const eng_half* gate, const eng_half* up, eng_half* out, int64_t n,
                   eng_stream stream) {
  return guarded([&] {
    ENG_CHECK(gate != nullptr, "swiglu_fp16: gate is null");
    ENG_CHECK(up != nullptr, "swiglu_fp16: up is null");
    ENG_CHECK(out != nullptr, "swiglu_fp16: out is null");
    ENG_CHECK(n >= 0, "swiglu_fp16: n must be non-negative");
    if (n == 0) return;
    hipStream_t s = eng::as_stream(stream);
    if (n % 8 == 0 && eng::aligned_to(gate, 16) && eng::aligned_to(up, 16) &&
        eng::aligned_to(out, 16)) {
      eng::swiglu_h8_kernel<<<eng::stream_grid(n / 8), eng::kThreads, 0, s>>>(
          reinterpret_cast<const eng::H8*>(gate), reinterpret_cast<const eng::H8*>(up),
          reinterpret_cast<eng::H8*>(out), n / 8);
    } else {
      eng::swiglu_h_scalar_kernel<<<eng::stream_grid(n), eng::kThreads, 0, s>>>(
          reinterpret_cast<const _Float16*>(gate), reinterpret_cast<const _Float16*>(up),
          reinterpret_cast<_Float16*>(out), n);
    }
    ENG_LAUNCH_CHECK();
  });
}

int eng_residual_rmsnorm_f32(const float* x, const float* residual, const float* weight,
                             float* norm_out, float* sum_out, int64_t rows, int64_t cols,
                             float eps, eng_stream stream) {
  return guarded([&] {
    ENG_CHECK(rows >= 0 && cols >= 0, "residual_rmsnorm: negative dimension");
    ENG_CHECK(x != nullptr && residual != nullptr && norm_out != nullptr && sum_out != nullptr,
              "residual_rmsnorm: null device pointer");
    ENG_CHECK(eps >= 0.0f, "residual_rmsnorm: eps must be non-negative");
    if (rows == 0 || cols == 0) return;
    hipStream_t s = eng::as_stream(stream);
    const long long wanted = 32LL * eng::device_cu_count();
    const unsigned grid = static_cast<unsigned>(std::min<long long>(rows, wanted));
    const bool vec = cols % 4 == 0 && eng::aligned_to(x, 16) && eng::aligned_to(residual, 16) &&
                     eng::aligned_to(norm_out, 16) && eng::aligned_to(sum_out, 16) &&
                     (weight == nullptr || eng::aligned_to(weight, 16));
    if (vec) {
      eng::residual_rmsnorm_kernel<true, 8><<<grid, eng::kThreads, 0, s>>>(
          x, residual, weight, norm_out, sum_out, rows, cols, eps);
    } else {
      eng::residual_rmsnorm_kernel<false, 16><<<grid, eng::kThreads, 0, s>>>(
          x, residual, weight, norm_out, sum_out, rows, cols, eps);
    }
    ENG_LAUNCH_CHECK();
  });
}

}  // extern "C"
