// gemv.hip -- split-K decode GEMV family for gfx950 (out[N] = x[K] . W[K x N]).
//
// Serves gemv (fp32 W), gemv_fp16 (half W/x/out), the fp16-weight / fp32-I/O
// overload and the M == 1 case of rmsnorm_linear (reference kernels/gemv.cu,
// kernels/gemv_fp16.cu, kernels/rmsnorm_linear.cu).
//
// Mapping (W row-major [K x N], rows contiguous along N):
//   * a workgroup owns a column block of CW = LPR * VEC columns and a chunk of
//     `kchunk` rows (split-K);
//   * inside a wave, LPR lanes cover one row segment with 16-byte loads (VEC
//     elements each) and the 64 / LPR lane groups read consecutive rows, so one
//     wave load instruction fetches 64 / LPR rows x (16 * LPR) contiguous bytes;
//     the 4 waves take the next rows, and the loop is unrolled so every lane has
//     kUnroll independent 16-byte loads in flight;
//   * partial sums are reduced across lane groups with cross-lane shuffles, then
//     across waves through LDS, then across split-K workgroups by the last
//     workgroup of each column block to arrive (arrival counter per column
//     block). The final sum runs over the splits in index order, so results do
//     not depend on scheduling.
// RMSNorm fusion: sum_k (x_k s g_k) W_kn = s * sum_k (x_k g_k) W_kn for the row
// scale s = 1/sqrt(mean(x^2) + eps), so the kernel streams W against x * gamma,
// accumulates sum x^2 over the rows it already reads, and applies s in the
// epilogue, after the split-K reduction has combined the per-split sums of squares.
#include "launch.hpp"

#include <algorithm>

namespace eng {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kUnroll = 8;

template <typename T>
__device__ __forceinline__ float to_f32(T v) {
  return static_cast<float>(v);
}

template <typename T>
__device__ __forceinline__ T from_f32(float v) {
  return static_cast<T>(v);  // float -> _Float16 rounds to nearest even
}

template <typename T, int VEC>
struct RawVec {
  typedef T type __attribute__((ext_vector_type(VEC)));
};
template <typename T>
struct RawVec<T, 1> {
  typedef T type;
};

template <int VEC, typename V>
__device__ __forceinline__ float lane_elem(const V& v, int e) {
  if constexpr (VEC == 1) {
    return static_cast<float>(v);
  } else {
    return static_cast<float>(v[e]);
  }
}

__device__ __forceinline__ void store_agent(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float load_agent(const float* p) {
  return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ float rms_scale(float sumsq, long long K, float eps) {
  return 1.0f / sqrtf(sumsq / static_cast<float>(K) + eps);
}

template <typename WT, typename XT, typename YT, int VEC, int LPR, bool RMS>
__global__ __launch_bounds__(kThreads) void gemv_splitk_kernel(
    const WT* __restrict__ W, const XT* __restrict__ x, const float* __restrict__ gamma,
    YT* __restrict__ y, long long N, long long K, long long kchunk, int nsplit,
    float* __restrict__ part, float* __restrict__ part_ss, unsigned* __restrict__ counters,
    float eps) {
  constexpr int RPW = 64 / LPR;       // rows per wave load
  constexpr int STEP = kWaves * RPW;  // rows per load of all waves
  constexpr int CW = LPR * VEC;       // columns per workgroup
  using V = typename RawVec<WT, VEC>::type;

  __shared__ float red[kWaves][CW];
  __shared__ float red_ss[kWaves];
  __shared__ unsigned sh_last;

  const int t = threadIdx.x;
  const int lane = t & 63;
  const int wave = t >> 6;
  const int seg = lane % LPR;
  const int rg = lane / LPR;
  const long long cb = blockIdx.x;
  const int s = blockIdx.y;
  const long long col0 = cb * CW + static_cast<long long>(seg) * VEC;
  const bool col_ok = col0 < N;  // VEC > 1 implies N % VEC == 0
  const long long row_begin = static_cast<long long>(s) * kchunk;
  const long long row_end = row_begin + kchunk < K ? row_begin + kchunk : K;

  float acc[VEC];
#pragma unroll
  for (int e = 0; e < VEC; ++e) acc[e] = 0.0f;
  float ss = 0.0f;

  const WT* wcol = W + col0;
  for (long long base = row_begin + wave * RPW + rg; base < row_end;
       base += static_cast<long long>(STEP) * kUnroll) {
    V raw[kUnroll];
    float xv[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const long long r = base + static_cast<long long>(u) * STEP;
      const bool ok = r < row_end;
      float xr = ok ? to_f32(x[r]) : 0.0f;
      if constexpr (RMS) {
        ss = fmaf(xr, xr, ss);
        if (gamma != nullptr && ok) xr *= gamma[r];
      }
      xv[u] = xr;
      raw[u] = (ok && col_ok) ? *reinterpret_cast<const V*>(wcol + r * N) : V{};
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
#pragma unroll
      for (int e = 0; e < VEC; ++e) acc[e] = fmaf(xv[u], lane_elem<VEC>(raw[u], e), acc[e]);
    }
  }

  // Lanes with the same `seg` hold the same columns: fold the row groups.
#pragma unroll
  for (int off = LPR; off < 64; off <<= 1) {
#pragma unroll
    for (int e = 0; e < VEC; ++e) acc[e] += __shfl_xor(acc[e], off);
    if constexpr (RMS) ss += __shfl_xor(ss, off);
  }
  if (rg == 0) {
#pragma unroll
    for (int e = 0; e < VEC; ++e) red[wave][seg * VEC + e] = acc[e];
  }
  if (RMS && lane == 0) red_ss[wave] = ss;
  __syncthreads();

  float wg_ss = 0.0f;
  if constexpr (RMS) {
#pragma unroll
    for (int w = 0; w < kWaves; ++w) wg_ss += red_ss[w];
  }

  if (nsplit == 1) {
    const float scale = RMS ? rms_scale(wg_ss, K, eps) : 1.0f;
    for (int c = t; c < CW; c += kThreads) {
      const long long col = cb * CW + c;
      if (col < N) {
        float v = red[0][c];
#pragma unroll
        for (int w = 1; w < kWaves; ++w) v += red[w][c];
        if constexpr (RMS) v *= scale;
        y[col] = from_f32<YT>(v);
      }
    }
    return;
  }

  // Publish this split's partial sums, then count arrivals for the column block.
  for (int c = t; c < CW; c += kThreads) {
    const long long col = cb * CW + c;
    if (col < N) {
      float v = red[0][c];
#pragma unroll
      for (int w = 1; w < kWaves; ++w) v += red[w][c];
      store_agent(&part[static_cast<long long>(s) * N + col], v);
    }
  }
  if (RMS && t == 0) store_agent(&part_ss[cb * nsplit + s], wg_ss);
  __threadfence();
  __syncthreads();
  if (t == 0) {
    const unsigned prev =
        __hip_atomic_fetch_add(&counters[cb], 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
    sh_last = (prev == static_cast<unsigned>(nsplit - 1)) ? 1u : 0u;
  }
  __syncthreads();
  if (sh_last == 0u) return;
  __threadfence();

  // Last arrival: combine the splits in index order.
  float scale = 1.0f;
  if constexpr (RMS) {
    float tot = 0.0f;
    for (int i = 0; i < nsplit; ++i) tot += load_agent(&part_ss[cb * nsplit + i]);
    scale = rms_scale(tot, K, eps);
  }
  for (int c = t; c < CW; c += kThreads) {
    const long long col = cb * CW + c;
    if (col < N) {
      float v = 0.0f;
#pragma unroll 8
      for (int i = 0; i < nsplit; ++i) v += load_agent(&part[static_cast<long long>(i) * N + col]);
      if constexpr (RMS) v *= scale;
      y[col] = from_f32<YT>(v);
    }
  }
  if (t == 0) __hip_atomic_store(&counters[cb], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <typename WT, typename XT, typename YT, int VEC, int LPR, bool RMS>
void run_gemv(const GemvArgs& a, hipStream_t stream) {
  constexpr int RPW = 64 / LPR;
  constexpr int STEP = kWaves * RPW;
  constexpr int CW = LPR * VEC;
  const long long N = a.N;
  const long long K = a.K;
  const long long ncb = (N + CW - 1) / CW;
  ENG_CHECK(ncb <= 0x7fffffffLL, "gemv: N too large for one launch");

  // Aim for ~4 workgroups per CU; never give a split fewer than STEP rows.
  const long long target = 4LL * device_cu_count();
  long long nsplit = (target + ncb - 1) / ncb;
  nsplit = std::min(nsplit, (K + STEP - 1) / STEP);
  nsplit = std::max(nsplit, 1LL);

  GemvWorkspace* ws = nullptr;
  if (nsplit > 1) {
    ws = &gemv_workspace(stream);
    if (ncb > static_cast<long long>(ws->capacity_counters)) {
      nsplit = 1;
    } else {
      nsplit = std::min(nsplit, static_cast<long long>(ws->capacity_partials) / N);
      nsplit = std::min(nsplit, static_cast<long long>(ws->capacity_ss) / ncb);
      nsplit = std::min(nsplit, 65535LL);
      nsplit = std::max(nsplit, 1LL);
    }
  }
  long long kchunk = (K + nsplit - 1) / nsplit;
  kchunk = (kchunk + STEP - 1) / STEP * STEP;
  nsplit = (K + kchunk - 1) / kchunk;

  dim3 grid(static_cast<unsigned>(ncb), static_cast<unsigned>(nsplit));
  gemv_splitk_kernel<WT, XT, YT, VEC, LPR, RMS><<<grid, kThreads, 0, stream>>>(
      static_cast<const WT*>(a.W), static_cast<const XT*>(a.x), a.gamma, static_cast<YT*>(a.y),
      N, K, kchunk, static_cast<int>(nsplit), ws ? ws->partials : nullptr,
      ws ? ws->partial_ss : nullptr, ws ? ws->counters : nullptr, a.eps);
  ENG_LAUNCH_CHECK();
}

// Row segments of 8 lanes x 16 bytes (128 B) for the vector paths; the scalar
// fallback (unaligned W or N not a multiple of the vector width) uses one lane
// per column.
template <typename WT, typename XT, typename YT, bool RMS>
void dispatch_vec(const GemvArgs& a, hipStream_t stream) {
  constexpr int VMAX = 16 / static_cast<int>(sizeof(WT));
  const bool vec_ok = (a.N % VMAX == 0) && aligned_to(a.W, 16);
  if (vec_ok) {
    run_gemv<WT, XT, YT, VMAX, 8, RMS>(a, stream);
  } else {
    run_gemv<WT, XT, YT, 1, 64, RMS>(a, stream);
  }
}

}  // namespace

int device_cu_count() {
  static int cached[64] = {0};
  int dev = 0;
  ENG_HIP_CHECK(hipGetDevice(&dev));
  if (dev >= 0 && dev < 64 && cached[dev] > 0) return cached[dev];
  int cus = 0;
  ENG_HIP_CHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
  if (cus <= 0) cus = 1;
  if (dev >= 0 && dev < 64) cached[dev] = cus;
  return cus;
}

void launch_gemv(const GemvArgs& a, hipStream_t stream) {
  if (a.w == Elem::F32) {
    ENG_CHECK(a.x_elem == Elem::F32 && a.y_elem == Elem::F32, "gemv: unsupported element types");
    if (a.rms) {
      dispatch_vec<float, float, float, true>(a, stream);
    } else {
      dispatch_vec<float, float, float, false>(a, stream);
    }
    return;
  }
  if (a.x_elem == Elem::F32 && a.y_elem == Elem::F32) {
    if (a.rms) {
      dispatch_vec<_Float16, float, float, true>(a, stream);
    } else {
      dispatch_vec<_Float16, float, float, false>(a, stream);
    }
    return;
  }
  ENG_CHECK(a.x_elem == Elem::F16 && a.y_elem == Elem::F16 && !a.rms,
            "gemv: unsupported element types");
  dispatch_vec<_Float16, _Float16, _Float16, false>(a, stream);
}

}  // namespace eng

using eng::guarded;

extern "C" {

int eng_gemv_f32(const float* A, const float* x, float* out, int64_t N, int64_t K,
                 eng_stream stream) {
  return guarded([&] {
    ENG_CHECK(A != nullptr, "gemv: A is null");
    ENG_CHECK(x != nullptr, "gemv: x is null");
    ENG_CHECK(out != nullptr, "gemv: out is null");
    ENG_CHECK(N >= 0, "gemv: N must be non-negative");
    ENG_CHECK(K >= 0, "gemv: K must be non-negative");
    if (N == 0) return;
    hipStream_t s = eng::as_stream(stream);
    // An empty dot product is zero: K == 0 yields an all-zero output.
    if (K == 0) {
      eng::fill_zero_async(out, static_cast<std::size_t>(N) * sizeof(float), s);
      return;
    }
    eng::GemvArgs a;
    a.W = A;
    a.w = eng::Elem::F32;
    a.x = x;
    a.y = out;
    a.N = N;
    a.K = K;
    eng::launch_gemv(a, s);
  });
}

int eng_gemv_f16(const eng_half* A, const eng_half* x, eng_half* out, int64_t N, int64_t K,
                 eng_stream stream) {
  return guarded([&] {
    ENG_CHECK(A != nullptr, "gemv_fp16: A is null");
    ENG_CHECK(x != nullptr, "gemv_fp16: x is null");
    ENG_CHECK(out != nullptr, "gemv_fp16: out is null");
    ENG_CHECK(N >= 0, "gemv_fp16: N must be non-negative");
    ENG_CHECK(K >= 0, "gemv_fp16: K must be non-negative");
    if (N == 0) return;
    hipStream_t s = eng::as_stream(stream);
    if (K == 0) {
      eng::fill_zero_async(out, static_cast<std::size_t>(N) * sizeof(eng_half), s);
      return;
    }
    eng::GemvArgs a;
    a.W = A;
    a.w = eng::Elem::F16;
    a.x = x;
    a.x_elem = eng::Elem::F16;
    a.y = out;
    a.y_elem = eng::Elem::F16;
    a.N = N;
    a.K = K;
    eng::launch_gemv(a, s);
  });
}

int eng_gemv_f16w(const eng_half* A, const float* x, float* out, int64_t N, int64_t K,
                  eng_stream stream) {
  return guarded([&] {
    ENG_CHECK(A != nullptr, "gemv_fp16: A is null");
    ENG_CHECK(x != nullptr, "gemv_fp16: x is null");
    ENG_CHECK(out != nullptr, "gemv_fp16: out is null");
    ENG_CHECK(N >= 0, "gemv_fp16: N must be non-negative");
    ENG_CHECK(K >= 0, "gemv_fp16: K must be non-negative");
    if (N == 0) return;
    hipStream_t s = eng::as_stream(stream);
    if (K == 0) {
      eng::fill_zero_async(out, static_cast<std::size_t>(N) * sizeof(float), s);
      return;
    }
    eng::GemvArgs a;
    a.W = A;
    a.w = eng::Elem::F16;
    a.x = x;
    a.y = out;
    a.N = N;
    a.K = K;
    eng::launch_gemv(a, s);
  });
}

}  // extern "C"
