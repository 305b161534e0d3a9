// gemv_kernels.hpp -- device code of the decode GEMV family (out[N] = x[K] . W[K x N]).
//
// Workgroup -> work mapping (W row-major [K x N], rows contiguous along N):
//   * a workgroup owns a column slab of CW = LPR * VEC columns and a range of
//     rows: all K rows (direct mode), or one of `nsplit` row chunks (partial
//     mode, for shapes with too few slabs to fill the GPU);
//   * inside a wave, LPR lanes cover one row segment with 16-byte loads (VEC
//     elements each) and the 64 / LPR lane groups take consecutive rows, so a
//     wave load instruction reads 64 / LPR rows x 16 * LPR bytes; the WAVES
//     waves take the following rows and the loop keeps U loads per lane in
//     flight;
//   * workgroups are handed to the 8 XCDs round-robin; the id -> slab map is
//     renumbered so each XCD walks a contiguous band of slabs, and slabs narrower
//     than a 128-byte line share their lines inside one XCD's L2.
// Sums are folded across lane groups with cross-lane shuffles and across waves
// through LDS, always in the same order (the output-major kernels below fold
// whole waves with wave_sum). Partial mode writes fp32 partial
// sums (and per-chunk sums of squares) that gemv_reduce_kernel combines in
// chunk order, so results never depend on scheduling and no workgroup waits
// on another.
// RMSNorm fusion: sum_k (x_k s g_k) W_kn = s * sum_k (x_k g_k) W_kn with the
// row scale s = 1/sqrt(mean(x^2) + eps): the kernel streams W against x * g,
// sums x^2 over the rows it reads anyway, and applies s last.
#pragma once

#include <hip/hip_runtime.h>

#include "device_sync.hpp"

namespace eng {
namespace gemv {

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

// x + (x of the lane that DPP control CTRL selects).
template <int CTRL>
__device__ __forceinline__ float dpp_add(float x) {
  const int y = __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xF, 0xF, false);
  return x + __builtin_bit_cast(float, y);
}

// Sum over the 64 lanes of a wave, in one fixed order, returned in every
// lane: DPP quad_perm xor-1 and xor-2, row_half_mirror (lane i <- 7 - i within
// 8 lanes) and row_mirror (i <- 15 - i) leave each 16-lane row's sum in all of
// its lanes (a + b == b + a, so both lanes of a pair hold the same bits); the
// four row sums, read from lanes 0, 16, 32 and 48, are added as
// (r0 + r1) + (r2 + r3). Four VALU adds and four lane reads, where a shuffle
// tree costs six LDS-crossbar round trips.
__device__ __forceinline__ float wave_sum(float x) {
  x = dpp_add<0xB1>(x);   // quad_perm [1, 0, 3, 2]
  x = dpp_add<0x4E>(x);   // quad_perm [2, 3, 0, 1]
  x = dpp_add<0x141>(x);  // row_half_mirror
  x = dpp_add<0x140>(x);  // row_mirror
  const int b = __builtin_bit_cast(int, x);
  const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 0));
  const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 16));
  const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 32));
  const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 48));
  return (r0 + r1) + (r2 + r3);
}

__device__ __forceinline__ float rms_scale(float sumsq, long long K, float eps) {
  return 1.0f / sqrtf(sumsq / static_cast<float>(K) + eps);
}

// SiLU(g) * u with SiLU(g) = g / (1 + e^-g) (reference src/cpu_ref/swiglu_cpu.cpp:
// 23-25): fp32 exp and a correctly rounded divide; large negative g gives
// g / inf = -0, large positive g gives g.
__device__ __forceinline__ float swiglu_f32(float g, float u) {
  return g / (1.0f + expf(-g)) * u;
}

// Workgroup id -> logical index so that XCD x (ids x, x + 8, ...) gets a
// contiguous range of logical indices. A bijection on [0, total).
__device__ __forceinline__ long long xcd_contiguous(long long wg, long long total) {
  constexpr long long kXcds = 8;
  const long long q = total / kXcds;
  const long long r = total % kXcds;
  const long long xcd = wg % kXcds;
  return xcd * q + (xcd < r ? xcd : r) + wg / kXcds;
}

// MX > 1: MX activation rows at once (small-batch decode), row m of x at
// x + m K and of y at y + m N; every weight row read is multiplied into all MX
// rows, each (m, column) summed in the single-row order, so row m equals a
// single-row call on x[m] bit for bit. Partial sums are laid out
// [nsplit][MX][N], sums of squares [nsplit][MX].
// DUAL (partial mode only): two matrices W and W2 of the same shape against
// the same x (an FFN's gate and up projections); ncb counts the column blocks
// of both -- blocks [0, ncb / 2) stream W, the rest the same columns of W2 --
// and partial sums are laid out [nsplit][MX][2][N]. Each block's arithmetic
// is the single-matrix kernel's.
template <typename WT, typename XT, typename YT, int VEC, int LPR, int WAVES, int U, bool NT,
          bool RMS, bool PARTIAL, int MX = 1, bool DUAL = false>
__global__ __launch_bounds__(WAVES * 64) void gemv_stream_kernel(
    const WT* __restrict__ W, const XT* __restrict__ x, const float* __restrict__ gamma,
    YT* __restrict__ y, long long N, long long K, long long kchunk, long long ncb,
    float* __restrict__ part, float* __restrict__ part_ss, float eps,
    const WT* __restrict__ W2) {
  static_assert(!DUAL || PARTIAL, "two matrices need the partial-sum reduce");
  constexpr int RPW = 64 / LPR;       // rows per wave load
  constexpr int STEP = WAVES * RPW;   // rows per load of all waves
  constexpr int CW = LPR * VEC;       // columns per workgroup
  constexpr int THREADS = WAVES * 64;
  using V = typename RawVec<WT, VEC>::type;

  __shared__ float red[MX][WAVES][CW];
  __shared__ float red_ss[MX][WAVES];

  const int t = threadIdx.x;
  const int lane = t & 63;
  const int wave = t >> 6;
  const int seg = lane % LPR;
  const int rg = lane / LPR;

  const long long total = static_cast<long long>(gridDim.x);
  const long long logical = xcd_contiguous(blockIdx.x, total);
  const long long cb_all = logical % ncb;
  const long long s = logical / ncb;
  const long long blocks_per_matrix = DUAL ? ncb / 2 : ncb;
  const bool upper = DUAL && cb_all >= blocks_per_matrix;  // streams W2
  const long long cb = upper ? cb_all - blocks_per_matrix : cb_all;

  const long long col0 = cb * CW + static_cast<long long>(seg) * VEC;
  const bool col_ok = col0 < N;  // VEC > 1 implies N % VEC == 0
  const long long row_begin = s * kchunk;
  const long long row_end = row_begin + kchunk < K ? row_begin + kchunk : K;

  float acc[MX][VEC];
  float ss[MX];
#pragma unroll
  for (int m = 0; m < MX; ++m) {
#pragma unroll
    for (int e = 0; e < VEC; ++e) acc[m][e] = 0.0f;
    ss[m] = 0.0f;
  }

  // Columns past N (whole vectors, as N % VEC == 0 when VEC > 1) read column
  // 0 instead; their sums are never written.
  const WT* wsafe = (upper ? W2 : W) + (col_ok ? col0 : 0);
  for (long long base = row_begin + wave * RPW + rg; base < row_end;
       base += static_cast<long long>(STEP) * U) {
    // All of a step's loads (W, x, gamma) are issued before any is used, and
    // none is conditional: rows past the chunk read its last row (in bounds)
    // and are zeroed where the products are formed. (Loads complete in
    // order, so using a value as soon as it is loaded -- or a conditional
    // load's register reused as the next address -- waits for every weight
    // load issued before it.)
    V raw[U];
    float xv[U][MX];
    float gv[U];
    bool okr[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const long long r = base + static_cast<long long>(u) * STEP;
      okr[u] = r < row_end;
      const long long rr = okr[u] ? r : row_end - 1;
#pragma unroll
      for (int m = 0; m < MX; ++m) xv[u][m] = to_f32(x[m * K + rr]);
      if constexpr (RMS) gv[u] = gamma != nullptr ? gamma[rr] : 1.0f;
      const V* p = reinterpret_cast<const V*>(wsafe + rr * N);
      if constexpr (NT) {
        raw[u] = __builtin_nontemporal_load(p);
      } else {
        raw[u] = *p;
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
#pragma unroll
      for (int m = 0; m < MX; ++m) {
        float xr = okr[u] ? xv[u][m] : 0.0f;
        if constexpr (RMS) {
          ss[m] = fmaf(xr, xr, ss[m]);
          xr *= gv[u];
        }
        const V w = okr[u] ? raw[u] : V{};
#pragma unroll
        for (int e = 0; e < VEC; ++e) acc[m][e] = fmaf(xr, lane_elem<VEC>(w, e), acc[m][e]);
      }
    }
  }

  // Lanes with the same `seg` hold the same columns: fold the row groups.
#pragma unroll
  for (int off = LPR; off < 64; off <<= 1) {
#pragma unroll
    for (int m = 0; m < MX; ++m) {
#pragma unroll
      for (int e = 0; e < VEC; ++e) acc[m][e] += __shfl_xor(acc[m][e], off);
      if constexpr (RMS) ss[m] += __shfl_xor(ss[m], off);
    }
  }
  if (rg == 0) {
#pragma unroll
    for (int m = 0; m < MX; ++m)
#pragma unroll
      for (int e = 0; e < VEC; ++e) red[m][wave][seg * VEC + e] = acc[m][e];
  }
  if (RMS && lane == 0) {
#pragma unroll
    for (int m = 0; m < MX; ++m) red_ss[m][wave] = ss[m];
  }
  __syncthreads();

  float wg_ss[MX];
  float scale[MX];
#pragma unroll
  for (int m = 0; m < MX; ++m) {
    wg_ss[m] = 0.0f;
    if constexpr (RMS) {
#pragma unroll
      for (int w = 0; w < WAVES; ++w) wg_ss[m] += red_ss[m][w];
    }
    scale[m] = (RMS && !PARTIAL) ? rms_scale(wg_ss[m], K, eps) : 1.0f;
  }

  for (int c = t; c < CW; c += THREADS) {
    const long long col = cb * CW + c;
    if (col < N) {
#pragma unroll
      for (int m = 0; m < MX; ++m) {
        float v = red[m][0][c];
#pragma unroll
        for (int w = 1; w < WAVES; ++w) v += red[m][w][c];
        if constexpr (PARTIAL) {
          if constexpr (DUAL) {
            part[((s * MX + m) * 2 + (upper ? 1 : 0)) * N + col] = v;
          } else {
            part[(s * MX + m) * N + col] = v;
          }
        } else {
          if constexpr (RMS) v *= scale[m];
          y[m * N + col] = from_f32<YT>(v);
        }
      }
    }
  }
  if constexpr (PARTIAL && RMS) {
    if (cb_all == 0 && t == 0) {
#pragma unroll
      for (int m = 0; m < MX; ++m) part_ss[s * MX + m] = wg_ss[m];
    }
  }
}

// y[col] = scale * sum_{s < nsplit} part[s][col]. A workgroup of
// kReduceWaves waves owns 64 columns; wave g sums the contiguous group of
// splits [g * per, (g + 1) * per) in split order with 8 loads in flight per
// lane (loads past the group re-read its last partial and add 0), and the
// group sums are added in group order, so the association is fixed for a
// given nsplit. Up to 64 splits take one round trip per lane (8 waves
// measured best: 4 or 16 were up to 0.4 us slower at 4096 x 4096 and
// 11008 x 4096). blockIdx.y selects the activation row m of an mx-row launch
// (partials [nsplit][mx][N], output row m at y + m N). GLU: partials
// [nsplit][mx][2][N] from the DUAL stream kernel (gate plane, then up), each
// plane summed exactly as a single matrix's, and y = SiLU(s g) * (s u).
constexpr int kReduceWaves = 8;

template <typename YT, bool RMS, int WAVES = kReduceWaves, bool GLU = false>
__global__ __launch_bounds__(WAVES * 64) void gemv_reduce_kernel(
    const float* __restrict__ part, const float* __restrict__ part_ss, YT* __restrict__ y,
    long long N, long long K, int nsplit, float eps, int mx) {
  constexpr int PLANES = GLU ? 2 : 1;
  __shared__ float group_sum[PLANES][WAVES][64];
  const int c = threadIdx.x & 63;
  const int g = threadIdx.x >> 6;
  const int m = blockIdx.y;
  const long long col = static_cast<long long>(blockIdx.x) * 64 + c;
  const long long cc = col < N ? col : N - 1;  // columns past N read column N - 1, never stored
  const int per = (nsplit + WAVES - 1) / WAVES;
  const int s0 = g * per < nsplit ? g * per : nsplit;
  const int s1 = s0 + per < nsplit ? s0 + per : nsplit;
  const float* pm = part + static_cast<long long>(m) * PLANES * N + cc;
  const long long stride = static_cast<long long>(mx) * PLANES * N;
  float v[PLANES];
#pragma unroll
  for (int q = 0; q < PLANES; ++q) v[q] = 0.0f;
  // RMS: the first sum-of-squares state of lane c (split c) is loaded ahead of
  // the partials and held past their loop (the asm), so with up to 64 splits
  // the scale costs no round trip after theirs (left to the compiler, the
  // load sank into wave 0's branch behind the partials' wait).
  [[maybe_unused]] float ss0 = 0.0f;
  if constexpr (RMS) ss0 = part_ss[static_cast<long long>(c < nsplit ? c : nsplit - 1) * mx + m];
  for (int s = s0; s < s1; s += 8) {
    float t[PLANES][8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int si = s + i < s1 ? s + i : s1 - 1;
#pragma unroll
      for (int q = 0; q < PLANES; ++q) t[q][i] = pm[static_cast<long long>(si) * stride + q * N];
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
#pragma unroll
      for (int q = 0; q < PLANES; ++q) v[q] += s + i < s1 ? t[q][i] : 0.0f;
    }
  }
  if constexpr (RMS) asm volatile("" : "+v"(ss0));
#pragma unroll
  for (int q = 0; q < PLANES; ++q) group_sum[q][g][c] = v[q];
  // Sum of squares over the splits: lane c of wave 0 takes splits c, c + 64,
  // ... in turn, then the lanes are folded (one fixed order per nsplit).
  float tot = 0.0f;
  if constexpr (RMS) {
    if (g == 0) {
      if (c < nsplit) tot += ss0;
      for (int s = c + 64; s < nsplit; s += 64) tot += part_ss[s * mx + m];
      tot = wave_sum(tot);
    }
  }
  __syncthreads();
  if (g != 0 || col >= N) return;
  float out[PLANES];
#pragma unroll
  for (int q = 0; q < PLANES; ++q) {
    out[q] = group_sum[q][0][c];
#pragma unroll
    for (int w = 1; w < WAVES; ++w) out[q] += group_sum[q][w][c];
    if constexpr (RMS) out[q] *= rms_scale(tot, K, eps);
  }
  if constexpr (GLU) {
    y[static_cast<long long>(m) * N + col] = from_f32<YT>(swiglu_f32(out[0], out[1]));
  } else {
    y[static_cast<long long>(m) * N + col] = from_f32<YT>(out[0]);
  }
}

// Output-major weights: y[n] = sum_k W[n][k] * xs[k] with W row-major [N x K]
// (xs = x * gamma, times the RMS row scale when RMS). Each wave owns R
// consecutive output rows; lane l reads 16-byte pieces l, l + 64, ... of each
// row (a wave load instruction is 1 KiB contiguous per row) together with the
// matching x values, keeps U steps of loads in flight, and folds its lanes
// with wave_sum at the end. No partial sums leave the wave. With RMS the wave
// also sums x^2 over the x values it reads anyway.
template <typename WT, int VEC, int R, int U, bool RMS>
__global__ __launch_bounds__(256) void gemv_rows_kernel(const WT* __restrict__ W,
                                                        const float* __restrict__ x,
                                                        const float* __restrict__ gamma,
                                                        float* __restrict__ y, long long N,
                                                        long long K, float eps) {
  using V = typename RawVec<WT, VEC>::type;
  using XV = typename RawVec<float, VEC>::type;
  constexpr int PIECE = 64 * VEC;  // elements per wave step
  const int lane = threadIdx.x & 63;
  const long long wave = (static_cast<long long>(blockIdx.x) * 256 + threadIdx.x) >> 6;
  const long long n0 = wave * R;
  if (n0 >= N) return;

  float acc[R];
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = 0.0f;
  float ss = 0.0f;
  const WT* rows[R];
#pragma unroll
  for (int r = 0; r < R; ++r) rows[r] = W + (n0 + r < N ? n0 + r : n0) * K;

  for (long long k0 = static_cast<long long>(lane) * VEC; k0 < K; k0 += static_cast<long long>(PIECE) * U) {
    V w[U][R];
    XV xv[U];
    XV gv[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const long long k = k0 + static_cast<long long>(u) * PIECE;
      const bool ok = k < K;  // VEC > 1 implies K % VEC == 0
#pragma unroll
      for (int r = 0; r < R; ++r) {
        // Weights are read once per call: nontemporal loads keep them from
        // displacing x (re-read by every wave) in the caches.
        if constexpr (VEC == 1) {
          w[u][r] = ok ? __builtin_nontemporal_load(rows[r] + k) : WT(0);
        } else {
          w[u][r] = ok ? __builtin_nontemporal_load(reinterpret_cast<const V*>(rows[r] + k)) : V{};
        }
      }
      if constexpr (VEC == 1) {
        xv[u] = ok ? x[k] : 0.0f;
        if constexpr (RMS) gv[u] = (ok && gamma != nullptr) ? gamma[k] : 1.0f;
      } else {
        xv[u] = ok ? *reinterpret_cast<const XV*>(x + k) : XV{};
        if constexpr (RMS) {
          if (gamma != nullptr && ok) {
            gv[u] = *reinterpret_cast<const XV*>(gamma + k);
          } else {
            gv[u] = XV{} + 1.0f;
          }
        }
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        float xe;
        float ge = 1.0f;
        if constexpr (VEC == 1) {
          xe = xv[u];
          if constexpr (RMS) ge = gv[u];
        } else {
          xe = xv[u][e];
          if constexpr (RMS) ge = gv[u][e];
        }
        if constexpr (RMS) {
          ss = fmaf(xe, xe, ss);
          xe *= ge;
        }
#pragma unroll
        for (int r = 0; r < R; ++r) acc[r] = fmaf(xe, lane_elem<VEC>(w[u][r], e), acc[r]);
      }
    }
  }
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = wave_sum(acc[r]);
  if constexpr (RMS) ss = wave_sum(ss);
  if (lane == 0) {
    const float scale = RMS ? rms_scale(ss, K, eps) : 1.0f;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      if (n0 + r < N) y[n0 + r] = RMS ? acc[r] * scale : acc[r];
    }
  }
}

// LDS slot of element k of the activation vector for the LDS-staged kernels.
// A wave step covers PIECE = 64 * VEC elements, lane l taking elements
// l*VEC .. l*VEC+VEC-1; the slot order stores, per piece, the first 4 of
// every lane's elements, then the next 4, so each 16-byte LDS read of a wave
// is contiguous across lanes (no bank conflicts). For VEC == 4 this is the
// identity.
template <int VEC>
__device__ __forceinline__ int lds_slot(int k) {
  constexpr int PIECE = 64 * VEC;
  const int p = k / PIECE;
  const int r = k - p * PIECE;
  const int l = r / VEC;
  const int e = r - l * VEC;
  return p * PIECE + (e >> 2) * 256 + l * 4 + (e & 3);
}

// Element index of the first of the 4 values at LDS float position pos (a
// multiple of 4): the inverse of lds_slot<VEC>.
template <int VEC>
__device__ __forceinline__ int slot_elem(int pos) {
  if constexpr (VEC == 4) {
    return pos;
  } else {
    const int p = pos >> 9;
    const int r = pos & 511;
    return p * 512 + ((r & 255) >> 2) * 8 + (r >> 8) * 4;
  }
}

// Workgroup-cooperative staging for the LDS kernels (THREADS threads) of MX
// activation rows (row m at x + m K, staged at xs + m pitch, its wave sums at
// wave_ss + 16 m): writes xs = x * gamma (gamma optional, applied only with
// RMS) into LDS slots, zero-padded to whole pieces, sums each row's x^2 (RMS)
// into total_ss[m], and ends with one barrier. K % 4 == 0 and 16-byte aligned
// x / gamma are required. Each row's arithmetic is the single row's.
// The sum has one fixed order for every workgroup size: 1024 virtual threads,
// v taking the 16-byte LDS positions v, v + 1024, v + 2048, ... in turn (each
// holding the 4 values slot_elem gives); each virtual wave (64 consecutive v)
// folded by wave_sum; the 16 virtual-wave sums added in order. (Positions
// rather than elements, so that the kernels staging x by direct-to-LDS loads
// -- wave w's load i filling positions 1024 i + 64 w .. + 63 -- can take the
// same sum from the values each thread loaded. A direct-staged RMSNorm
// GEMV built that way, gamma staged beside x and multiplied in as each wave
// reads it, ran config 3 in 16.1-16.3 us against 15.7-15.8 for this staging.) A workgroup of THREADS threads plays virtual threads tid,
// tid + THREADS, ..., so kernels with different workgroup sizes (and the
// small-batch kernels, which stage row by row) compute the same bits.
// wave_ss holds kStageWaves floats of shared memory.
constexpr int kStageWaves = 16;

// Makes v be computed here: the sum of the per-wave sums of squares is read
// from LDS right after the staging barrier instead of where the scale is used
// after the row stream, where the reads wait behind the other waves' LDS
// reads (the fused gate / up: 27.6 us against 27.8-28.4 deferred).
__device__ __forceinline__ void pin_here(float& v) {
  asm volatile("" : "+v"(v));
  __builtin_amdgcn_sched_barrier(0);
}

template <int VEC, bool RMS, int THREADS, int MX>
__device__ __forceinline__ void stage_xs_rows(const float* __restrict__ x,
                                              const float* __restrict__ gamma, long long K,
                                              int npieces, float* xs, int pitch,
                                              float* wave_ss, float* total_ss) {
  static_assert(THREADS == 256 || THREADS == 512 || THREADS == 1024, "4, 8 or 16 waves");
  using F4 = typename RawVec<float, 4>::type;
  constexpr int PIECE = 64 * VEC;
  constexpr int VT = kStageWaves * 64;  // virtual threads
  constexpr int JV = VT / THREADS;      // virtual threads per thread
  const int tid = threadIdx.x;
  float ss[MX][JV];
#pragma unroll
  for (int m = 0; m < MX; ++m)
#pragma unroll
    for (int j = 0; j < JV; ++j) ss[m][j] = 0.0f;
  const int padded = npieces * PIECE;
  // A round's x and gamma loads (every row's x, gamma once) are all issued
  // before any is used (in-bounds offsets: positions past K read element 0
  // and store zeros), so the staging waits once per round, not once per load
  // or per row.
  const float* gp = (RMS && gamma != nullptr) ? gamma : x;
  for (int base = 0; base < padded; base += VT * 4) {
    F4 xv[MX][JV];
    [[maybe_unused]] F4 gv[JV];
#pragma unroll
    for (int j = 0; j < JV; ++j) {
      const int pos = base + (tid + j * THREADS) * 4;
      const int k = pos < padded ? slot_elem<VEC>(pos) : 0;
      const int kc = k < K ? k : 0;
#pragma unroll
      for (int m = 0; m < MX; ++m) xv[m][j] = *reinterpret_cast<const F4*>(x + m * K + kc);
      if constexpr (RMS) gv[j] = *reinterpret_cast<const F4*>(gp + kc);
    }
    __builtin_amdgcn_sched_barrier(0);  // every load issued before the first use
#pragma unroll
    for (int j = 0; j < JV; ++j) {
      const int pos = base + (tid + j * THREADS) * 4;
      if (pos < padded) {
        const int k = slot_elem<VEC>(pos);
        const bool in = k < K;
#pragma unroll
        for (int m = 0; m < MX; ++m) {
          // Branch-free (selects), so the gamma load is not sunk into a
          // branch behind the wait for x: positions past K square and store
          // zeros (adding 0 * 0 leaves a sum of squares unchanged).
          F4 v = in ? xv[m][j] : F4{};
          if constexpr (RMS) {
            ss[m][j] = fmaf(v[0], v[0], ss[m][j]);
            ss[m][j] = fmaf(v[1], v[1], ss[m][j]);
            ss[m][j] = fmaf(v[2], v[2], ss[m][j]);
            ss[m][j] = fmaf(v[3], v[3], ss[m][j]);
            const F4 g = gamma != nullptr ? gv[j] : F4{1.0f, 1.0f, 1.0f, 1.0f};
            v = in ? v * g : F4{};
          }
          *reinterpret_cast<F4*>(xs + m * pitch + pos) = v;
        }
      }
    }
  }
  if constexpr (RMS) {
#pragma unroll
    for (int m = 0; m < MX; ++m) {
#pragma unroll
      for (int j = 0; j < JV; ++j) {
        const float w = wave_sum(ss[m][j]);
        if ((tid & 63) == 0) wave_ss[m * kStageWaves + (tid >> 6) + j * (THREADS / 64)] = w;
      }
    }
  }
  __syncthreads();
  if constexpr (RMS) {
#pragma unroll
    for (int m = 0; m < MX; ++m) {
      float t = wave_ss[m * kStageWaves];
#pragma unroll
      for (int w = 1; w < kStageWaves; ++w) t += wave_ss[m * kStageWaves + w];
      pin_here(t);
      total_ss[m] = t;
    }
  }
}

// One activation row: stage_xs_rows with MX = 1.
template <int VEC, bool RMS, int THREADS = 256>
__device__ __forceinline__ void stage_xs(const float* __restrict__ x,
                                         const float* __restrict__ gamma, long long K,
                                         int npieces, float* xs, float* wave_ss,
                                         float* total_ss) {
  stage_xs_rows<VEC, RMS, THREADS, 1>(x, gamma, K, npieces, xs, 0, wave_ss, total_ss);
}

// acc[j] = sum_k rows[j][k] * xs[k]: each lane sums its elements, then
// wave_sum folds the lanes (the result is in every lane). NR weight rows
// streamed with 16-byte nontemporal loads, U loads per row in flight, against
// the staged vector in LDS. Each lane's order is gemv_rows_kernel's, so the
// register and LDS kernels agree bit for bit without RMSNorm.
template <typename WT, int VEC, int NR, int U>
__device__ __forceinline__ void dot_rows_lds(const WT* const (&rows)[NR], const float* xs,
                                             long long K, int npieces, int lane,
                                             float (&acc)[NR]) {
  using V = typename RawVec<WT, VEC>::type;
  using F4 = typename RawVec<float, 4>::type;
  constexpr int PIECE = 64 * VEC;
#pragma unroll
  for (int j = 0; j < NR; ++j) acc[j] = 0.0f;
  for (int p0 = 0; p0 < npieces; p0 += U) {
    V cur[U][NR];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const long long k = static_cast<long long>(p0 + u) * PIECE + lane * VEC;
      const bool ok = k < K;
#pragma unroll
      for (int j = 0; j < NR; ++j) {
        cur[u][j] = ok ? __builtin_nontemporal_load(reinterpret_cast<const V*>(rows[j] + k)) : V{};
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (p0 + u >= npieces) break;  // wave-uniform
      const float* base = xs + (p0 + u) * PIECE + lane * 4;
#pragma unroll
      for (int h = 0; h < VEC / 4; ++h) {
        const F4 a = *reinterpret_cast<const F4*>(base + h * 256);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
#pragma unroll
          for (int j = 0; j < NR; ++j) {
            acc[j] = fmaf(a[e], static_cast<float>(cur[u][j][h * 4 + e]), acc[j]);
          }
        }
      }
    }
  }
#pragma unroll
  for (int j = 0; j < NR; ++j) acc[j] = wave_sum(acc[j]);
}

// dot_rows_lds for a K fixed at compile time, K = (NP - 1) * PIECE + KT with
// 0 < KT <= PIECE (the launchers instantiate it for common model widths).
// The pieces go in groups of CH with all of a group's loads in flight before
// any is used; every group but the last runs in a loop the compiler may not
// unroll, ending in a scheduling barrier (so later groups' loads cannot be
// hoisted and spill), and only the last piece, when partial, is masked (lanes
// past K read nothing). With K a
// runtime value every load needs a mask (an exec-mask branch per load) and
// the loop a trip-count test: the fixed form is 0.5-0.8 us faster per launch
// at the decode shapes. The arithmetic -- pieces in order, then the 4-float
// LDS groups, then elements -- is dot_rows_lds's, so the results are its bits.
template <typename WT, int VEC, int NR, int NP, int KT, int CH>
__device__ __forceinline__ void dot_rows_lds_fixed(const WT* const (&rows)[NR], const float* xs,
                                                   int lane, float (&acc)[NR]) {
  using V = typename RawVec<WT, VEC>::type;
  using F4 = typename RawVec<float, 4>::type;
  constexpr int PIECE = 64 * VEC;
  static_assert(NP >= 1 && KT > 0 && KT <= PIECE && KT % VEC == 0, "K = (NP - 1) * PIECE + KT");
  static_assert(CH >= 1 && CH <= NP, "group size");
  constexpr int G = (NP + CH - 1) / CH;     // groups of pieces
  constexpr int LAST = NP - (G - 1) * CH;   // pieces in the last group
#pragma unroll
  for (int j = 0; j < NR; ++j) acc[j] = 0.0f;
  const int lk = lane * VEC;
  auto use = [&](int p, const V (&w)[NR]) {
    const float* base = xs + p * PIECE + lane * 4;
#pragma unroll
    for (int h = 0; h < VEC / 4; ++h) {
      const F4 a = *reinterpret_cast<const F4*>(base + h * 256);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
#pragma unroll
        for (int j = 0; j < NR; ++j) acc[j] = fmaf(a[e], static_cast<float>(w[j][h * 4 + e]), acc[j]);
      }
    }
  };
#pragma unroll 1
  for (int c = 0; c < G - 1; ++c) {
    V cur[CH][NR];
#pragma unroll
    for (int u = 0; u < CH; ++u) {
#pragma unroll
      for (int j = 0; j < NR; ++j)
        cur[u][j] = __builtin_nontemporal_load(
            reinterpret_cast<const V*>(rows[j] + (c * CH + u) * PIECE + lk));
    }
#pragma unroll
    for (int u = 0; u < CH; ++u) use(c * CH + u, cur[u]);
    // Nothing moves across: a loop of one group is straight-line code, and
    // the next group's loads hoisted above this one's use would spill.
    __builtin_amdgcn_sched_barrier(0);
  }
  {
    constexpr int P0 = (G - 1) * CH;
    V cur[LAST][NR];
#pragma unroll
    for (int u = 0; u < LAST; ++u) {
      const bool ok = P0 + u < NP - 1 || KT == PIECE || lk < KT;  // only a partial last piece is masked
#pragma unroll
      for (int j = 0; j < NR; ++j)
        cur[u][j] = ok ? __builtin_nontemporal_load(
                             reinterpret_cast<const V*>(rows[j] + (P0 + u) * PIECE + lk))
                       : V{};
    }
#pragma unroll
    for (int u = 0; u < LAST; ++u) use(P0 + u, cur[u]);
  }
#pragma unroll
  for (int j = 0; j < NR; ++j) acc[j] = wave_sum(acc[j]);
}

// Output-major GEMV with the activation vector staged once per workgroup.
// Same arithmetic contract as gemv_rows_kernel (y[n] = s * sum_k W[n][k] *
// x[k] * g[k]), for when x (and gamma) are too large to stay in the vector L1
// across the rows a CU streams: the workgroup stages x * gamma in LDS
// (stage_xs), then each wave streams its R rows against LDS, U loads per row
// in flight (dot_rows_lds). (Issuing weight loads ahead of the staging
// measured slower: vector loads complete in order, so the staging then waits
// for HBM.) Workgroups of WAVES waves: 16 (one workgroup of 1024 threads per
// 16 rows) stages x once per 16 rows instead of once per 4 and lets the LDS
// budget hold twice the resident waves. Requires K % VEC == 0 and 16-byte
// aligned W, x and gamma; the caller sizes dynamic LDS as round_up(K, 64 *
// VEC) floats.
// NP > 0: K is the compile-time (NP - 1) * 64 VEC + KT (the caller checks
// it) and the rows stream through dot_rows_lds_fixed, CH pieces at a time.
template <typename WT, int VEC, int R, int U, bool RMS, int WAVES = 4, int NP = 0, int KT = 0,
          int CH = 0>
__global__ __launch_bounds__(WAVES * 64) void gemv_rows_lds_kernel(const WT* __restrict__ W,
                                                            const float* __restrict__ x,
                                                            const float* __restrict__ gamma,
                                                            float* __restrict__ y, long long N,
                                                            long long K, float eps) {
  static_assert(VEC == 4 || VEC == 8, "16-byte weight loads");
  constexpr int PIECE = 64 * VEC;
  extern __shared__ float xs[];
  __shared__ float wave_ss[kStageWaves];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const long long n0 = (static_cast<long long>(blockIdx.x) * WAVES + wave) * R;
  const int npieces = NP > 0 ? NP : static_cast<int>((K + PIECE - 1) / PIECE);

  float total_ss = 0.0f;
  stage_xs<VEC, RMS, WAVES * 64>(x, gamma, K, npieces, xs, wave_ss, &total_ss);
  if (n0 >= N) return;

  const WT* rows[R];
#pragma unroll
  for (int r = 0; r < R; ++r) rows[r] = W + (n0 + r < N ? n0 + r : n0) * K;
  float acc[R];
  if constexpr (NP > 0) {
    dot_rows_lds_fixed<WT, VEC, R, NP, KT, CH>(rows, xs, lane, acc);
  } else {
    dot_rows_lds<WT, VEC, R, U>(rows, xs, K, npieces, lane, acc);
  }
  if (lane == 0) {
    const float scale = RMS ? rms_scale(total_ss, K, eps) : 1.0f;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      if (n0 + r < N) y[n0 + r] = RMS ? acc[r] * scale : acc[r];
    }
  }
}


// Persistent form of gemv_rows_lds_kernel<_Float16, 8, 1, 4, RMS, 16, NP, KT,
// NP> for more rows than one resident round (two 16-wave workgroups per CU):
// a grid of P workgroups stages x * gamma once each, and wave w of workgroup
// b takes rows 16 b + w, then + 16 P, ... (a workgroup's waves read 16
// consecutive rows, as in the staged kernel). Its row's NP pieces (all of a
// row of K <= 4096) sit in a ring: the registers of piece p take piece p of
// the wave's next row right after the use that frees them, so the next row
// streams in while this one is summed -- no second round of workgroups, whose
// staging would start late. At 11008 x 4096 with RMSNorm 15.3 us against
// 15.8-15.9 staged (12288 rows: 16.8 against 17.1-17.2); loading the next row
// only after summing this one ran 22.8 us, and rows w P + b per wave (16 rows
// 4 MiB apart per workgroup) 17.0 us with the ring. Each row's sum is the
// staged kernel's (pieces in order, then the 4-float LDS groups, then
// elements) with the same scale: the same bits. Dynamic LDS: NP * 512 floats.
template <int NP, int KT, bool RMS>
__global__ __launch_bounds__(1024) void gemv_rows_persist_kernel(const _Float16* __restrict__ W,
                                                                  const float* __restrict__ x,
                                                                  const float* __restrict__ gamma,
                                                                  float* __restrict__ y,
                                                                  long long N, float eps) {
  using V = typename RawVec<_Float16, 8>::type;
  using F4 = typename RawVec<float, 4>::type;
  constexpr int PIECE = 512;
  constexpr int K = (NP - 1) * PIECE + KT;
  constexpr int WAVES = kStageWaves;
  static_assert(KT > 0 && KT <= PIECE && KT % 8 == 0, "K = (NP - 1) * 512 + KT");
  static_assert(NP >= 1 && NP <= 8, "a ring of the row's pieces (K <= 4096)");
  extern __shared__ float xs[];
  __shared__ float wave_ss[kStageWaves];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const long long stride = static_cast<long long>(WAVES) * gridDim.x;
  long long r = static_cast<long long>(blockIdx.x) * WAVES + wave;

  float total_ss = 0.0f;
  stage_xs<8, RMS, WAVES * 64>(x, gamma, K, NP, xs, wave_ss, &total_ss);
  const float scale = RMS ? rms_scale(total_ss, K, eps) : 1.0f;
  if (r >= N) return;  // no barrier follows

  const int lk = lane * 8;
  auto ok = [&](int p) { return p < NP - 1 || KT == PIECE || lk < KT; };
  auto load = [&](const _Float16* row, int p) -> V {
    return __builtin_nontemporal_load(
        reinterpret_cast<const V*>(row + p * PIECE + (ok(p) ? lk : 0)));
  };
  auto use = [&](int p, const V& w, float& acc) {
    const float* base = xs + p * PIECE + lane * 4;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const F4 a = *reinterpret_cast<const F4*>(base + h * 256);
#pragma unroll
      for (int e = 0; e < 4; ++e) acc = fmaf(a[e], static_cast<float>(w[h * 4 + e]), acc);
    }
  };
  V ring[NP];
#pragma unroll
  for (int p = 0; p < NP; ++p) ring[p] = load(W + r * K, p);
  for (;;) {
    const long long rn = r + stride;
    float acc = 0.0f;
    if (rn < N) {  // wave-uniform
      const _Float16* next = W + rn * K;
#pragma unroll
      for (int p = 0; p < NP; ++p) {
        use(p, ok(p) ? ring[p] : V{}, acc);
        ring[p] = load(next, p);
        // the reload stays right after the use that frees its registers
        asm volatile("" ::: "memory");
        __builtin_amdgcn_sched_barrier(0);
      }
    } else {
#pragma unroll
      for (int p = 0; p < NP; ++p) use(p, ok(p) ? ring[p] : V{}, acc);
    }
    acc = wave_sum(acc);
    if (lane == 0) y[r] = RMS ? acc * scale : acc;
    if (rn >= N) break;
    r = rn;
  }
}

// Output-major fp16 GEMV (no RMSNorm) for K fixed at compile time
// (K = (NP - 1) * 512 + KT), workgroups of 16 waves, one row per wave: the
// arithmetic of gemv_rows_lds_kernel<_Float16, 8, 1, 4, false, 16, NP, KT, CH>
// -- the same bits -- with x staged by direct global -> LDS loads issued
// together with the row's first weight loads: a thread issues its staging
// loads, then its wave's first CH weight pieces, and only then waits for the
// staging (vmcnt counts its weight loads out) and meets the other waves at a
// barrier without a fence, so the weight stream starts at once instead of
// after the staging round trip. The LDS slot layout is lds_slot<8>: each
// 16-byte chunk of it is 4 consecutive elements of x, so a lane fetches the
// chunk its LDS position holds; chunks past K are zeroed with LDS stores.
// (With RMSNorm, staging x this way needs a second barrier for the sum of
// squares and measured 2% slower at 11008 x 4096; gemv_rows_rms_early_kernel
// starts the weight stream early with register staging instead, for the
// fused gate / up.)
// Dynamic LDS: NP * 512 floats.
template <int NP, int KT, int CH, int WAVES = 16>
__global__ __launch_bounds__(64 * WAVES) void gemv_rows_dma_kernel(const _Float16* __restrict__ W,
                                                             const float* __restrict__ x,
                                                             float* __restrict__ y, long long N) {
  using V = typename RawVec<_Float16, 8>::type;
  using F4 = typename RawVec<float, 4>::type;
  constexpr int PIECE = 512;
  constexpr int K = (NP - 1) * PIECE + KT;
  constexpr int CHUNKS = NP * PIECE / 4;           // 16-byte chunks of the staged vector
  constexpr int NT = 64 * WAVES;
  constexpr int INSTR = (CHUNKS + NT - 1) / NT;    // staging loads per thread
  constexpr int G = (NP + CH - 1) / CH;
  constexpr int LAST = NP - (G - 1) * CH;
  static_assert(KT > 0 && KT <= PIECE && KT % 8 == 0, "K = (NP - 1) * 512 + KT");
  static_assert(CH >= 1 && CH <= NP, "groups of 1 to NP pieces");
  extern __shared__ float xs[];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const long long n0 = static_cast<long long>(blockIdx.x) * WAVES + wave;

  // Staging: wave w's i-th load fills chunks (WAVES i + w) * 64 .. + 63 of the
  // LDS vector; chunk q holds elements chunk_k0(q) .. + 3 of x. Chunks past K
  // (the last piece when KT < 512) are zeroed first, with LDS stores (a store
  // after a direct load the compiler cannot prove disjoint would make it
  // wait for the load).
  auto chunk_k0 = [](int q) {
    const int p = q >> 7;
    const int r = q & 127;
    return p * PIECE + (r & 63) * 8 + (r >> 6) * 4;
  };
  if constexpr (KT < PIECE) {
#pragma unroll
    for (int i = 0; i < INSTR; ++i) {
      const int q = (WAVES * i + wave) * 64 + lane;
      if (q < CHUNKS && chunk_k0(q) >= K) *reinterpret_cast<F4*>(xs + 4 * q) = F4{};
    }
  }
#pragma unroll
  for (int i = 0; i < INSTR; ++i) {
    const int q0 = (WAVES * i + wave) * 64;
    if (q0 < CHUNKS) {  // wave-uniform
      const int q = q0 + lane;
      if (q < CHUNKS && chunk_k0(q) < K) dma16(x + chunk_k0(q), xs + 4 * q0);
    }
  }
  // The staging loads must be issued before the weight loads: the wait below
  // counts the weight loads out, and loads complete in issue order.
  __builtin_amdgcn_sched_barrier(0);

  const bool active = n0 < N;
  const _Float16* row = W + (active ? n0 : N - 1) * static_cast<long long>(K);
  const int lk = lane * 8;
  float acc = 0.0f;
  auto use = [&](int p, const V& w) {
    const float* base = xs + p * PIECE + lane * 4;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const F4 a = *reinterpret_cast<const F4*>(base + h * 256);
#pragma unroll
      for (int e = 0; e < 4; ++e) acc = fmaf(a[e], static_cast<float>(w[h * 4 + e]), acc);
    }
  };
  // A partial last piece is loaded by every lane (lanes past K read the
  // piece's first 16 bytes, in bounds) and zeroed where it is used: no branch
  // around a load, and nothing that needs the data before the first wait (a
  // branch or an early select there makes the compiler wait for every load).
  auto ok = [&](int p) { return p < NP - 1 || KT == PIECE || lk < KT; };
  auto load = [&](int p) -> V {
    return __builtin_nontemporal_load(reinterpret_cast<const V*>(row + p * PIECE + (ok(p) ? lk : 0)));
  };

  // First group of weight pieces, then wait for the staging only.
  {
    constexpr int FIRST = G > 1 ? CH : LAST;
    V cur[FIRST];
#pragma unroll
    for (int u = 0; u < FIRST; ++u) cur[u] = load(u);
#if defined(__HIP_DEVICE_COMPILE__)
    // loads complete in order: at most FIRST (this wave's weight loads)
    // outstanding means the staging loads have landed; the zero stores of
    // padding chunks must be done too
    __builtin_amdgcn_s_waitcnt(vmcnt_le(FIRST));
    __builtin_amdgcn_s_waitcnt(lgkmcnt_zero());
#endif
    __builtin_amdgcn_sched_barrier(0);
    barrier_no_fence();
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < FIRST; ++u) use(u, ok(u) ? cur[u] : V{});
    __builtin_amdgcn_sched_barrier(0);
  }
  // Whole groups of CH pieces, then (when CH does not divide NP) the last
  // LAST pieces: no load past piece NP - 1.
  constexpr int FULL = LAST == CH ? G : G - 1;
#pragma unroll 1
  for (int c = 1; c < FULL; ++c) {
    V cur[CH];
#pragma unroll
    for (int u = 0; u < CH; ++u) cur[u] = load(c * CH + u);
#pragma unroll
    for (int u = 0; u < CH; ++u) use(c * CH + u, ok(c * CH + u) ? cur[u] : V{});
    __builtin_amdgcn_sched_barrier(0);
  }
  if constexpr (FULL < G && G > 1) {
    constexpr int P0 = (G - 1) * CH;
    V cur[LAST];
#pragma unroll
    for (int u = 0; u < LAST; ++u) cur[u] = load(P0 + u);
#pragma unroll
    for (int u = 0; u < LAST; ++u) use(P0 + u, ok(P0 + u) ? cur[u] : V{});
  }
  acc = wave_sum(acc);
  if (lane == 0 && active) y[n0] = acc;
}

// Fixed-K fp16 fused gate / up + SwiGLU (GLU = true: y[n] = SiLU(s Wg[n] .
// xs) * (s Wu[n] . xs)) or RMSNorm GEMV (GLU = false: y[n] = s W[n] . xs; not
// dispatched: it ran 15.5 us at 11008 x 4096 on some boxes and 17.5 on others,
// against 15.8-15.9 for the staged kernel),
// xs = x * gamma, K = (NP - 1) * 512 + KT, 16-wave workgroups, one output per
// wave: the bits of gemv_rows_lds_kernel<_Float16, 8, 1, 4, true, 16, NP, KT,
// CH> (GLU: gemv_rows_glu_kernel<...>), with the weight stream started before
// the staging completes and kept at CH pieces per row in flight (a ring: the
// registers of a used piece take the piece CH further on; GLU streams two
// rows, so CH = 4 keeps its 16 waves at 64 VGPRs, two workgroups per CU).
// Each thread loads its x and gamma chunks (the LDS positions
// stage_xs gives virtual thread tid, so the sum of squares has stage_xs's
// order), then its wave's first CH weight pieces per row, and only then
// waits for its x and gamma, writes x * gamma to LDS and its wave's sum of
// squares, and meets the other waves at one barrier without a fence (a
// fence would wait for the weights). Loads complete in issue order, so the
// wait for x and gamma leaves the weight loads in flight. All loads use
// in-bounds offsets (chunks past K read chunk 0, weight lanes past K the
// piece's first 16 bytes) and are zeroed where used: no branch or select
// between a load and the wait; every thread stores its chunk, so the LDS
// vector is rounded up to whole rounds of 1024 chunks (the slots past NP
// pieces are written and never read).
// Dynamic LDS: rms_early_lds_floats(NP) floats.
constexpr int rms_early_lds_floats(int np) { return (np * 512 + 4095) / 4096 * 4096; }

template <int NP, int KT, int CH, bool GLU>
__global__ __launch_bounds__(1024) void gemv_rows_rms_early_kernel(
    const _Float16* __restrict__ W0, const _Float16* __restrict__ W1,
    const float* __restrict__ x, const float* __restrict__ gamma, float* __restrict__ y,
    long long N, float eps) {
  using V = typename RawVec<_Float16, 8>::type;
  using F4 = typename RawVec<float, 4>::type;
  constexpr int PIECE = 512;
  constexpr int K = (NP - 1) * PIECE + KT;
  constexpr int VT = kStageWaves * 64;            // stage_xs's virtual threads: one per thread
  constexpr int ITER = rms_early_lds_floats(NP) / (VT * 4);
  constexpr int NR = GLU ? 2 : 1;
  static_assert(KT > 0 && KT <= PIECE && KT % 8 == 0, "K = (NP - 1) * 512 + KT");
  static_assert(CH >= 1 && CH <= NP, "ring of 1 to NP pieces");
  extern __shared__ float xs[];
  __shared__ float wave_ss[kStageWaves];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const long long n0 = static_cast<long long>(blockIdx.x) * kStageWaves + wave;

  // Staging loads: x and gamma chunk i * VT + tid (gamma == nullptr: x again,
  // read as 1 below).
  const float* gp = gamma != nullptr ? gamma : x;
  F4 xv[ITER], gv[ITER];
#pragma unroll
  for (int i = 0; i < ITER; ++i) {
    const int k = slot_elem<8>((i * VT + tid) * 4);
    const int kc = k < K ? k : 0;
    xv[i] = *reinterpret_cast<const F4*>(x + kc);
    gv[i] = *reinterpret_cast<const F4*>(gp + kc);
  }
  __builtin_amdgcn_sched_barrier(0);

  const bool active = n0 < N;
  const long long nr = active ? n0 : N - 1;
  const _Float16* rows[NR];
  rows[0] = W0 + nr * K;
  if constexpr (GLU) rows[1] = W1 + nr * K;
  const int lk = lane * 8;
  auto ok = [&](int p) { return p < NP - 1 || KT == PIECE || lk < KT; };
  auto load = [&](int j, int p) -> V {
    return __builtin_nontemporal_load(
        reinterpret_cast<const V*>(rows[j] + p * PIECE + (ok(p) ? lk : 0)));
  };
  float acc[NR];
#pragma unroll
  for (int j = 0; j < NR; ++j) acc[j] = 0.0f;
  auto use = [&](int p, const V (&w)[NR]) {
    const float* base = xs + p * PIECE + lane * 4;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const F4 a = *reinterpret_cast<const F4*>(base + h * 256);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
#pragma unroll
        for (int j = 0; j < NR; ++j) acc[j] = fmaf(a[e], static_cast<float>(w[j][h * 4 + e]), acc[j]);
      }
    }
  };

  // Ring of the next CH pieces (per row): pieces 0 .. CH - 1 now, piece
  // p + CH loaded once piece p is used.
  V ring[CH][NR];
#pragma unroll
  for (int u = 0; u < CH; ++u) {
#pragma unroll
    for (int j = 0; j < NR; ++j) ring[u][j] = load(j, u);
  }
  __builtin_amdgcn_sched_barrier(0);

  // x * gamma into LDS (zero past K), the sum of squares in stage_xs's order.
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < ITER; ++i) {
    const int pos = (i * VT + tid) * 4;
    const int k = slot_elem<8>(pos);
    F4 v = k < K ? xv[i] : F4{};
    ss = fmaf(v[0], v[0], ss);
    ss = fmaf(v[1], v[1], ss);
    ss = fmaf(v[2], v[2], ss);
    ss = fmaf(v[3], v[3], ss);
    if (gamma != nullptr) v *= gv[i];
    *reinterpret_cast<F4*>(xs + pos) = v;
  }
  ss = wave_sum(ss);
  if (lane == 0) wave_ss[wave] = ss;
  lds_barrier();
  float total = wave_ss[0];
#pragma unroll
  for (int w = 1; w < kStageWaves; ++w) total += wave_ss[w];
  pin_here(total);
  const float scale = rms_scale(total, K, eps);

#pragma unroll
  for (int p = 0; p < NP; ++p) {
    V w[NR];
#pragma unroll
    for (int j = 0; j < NR; ++j) w[j] = ok(p) ? ring[p % CH][j] : V{};
    use(p, w);
    if (p + CH < NP) {
#pragma unroll
      for (int j = 0; j < NR; ++j) ring[p % CH][j] = load(j, p + CH);
    }
    // each load issued right after the use that frees its registers, and no
    // later LDS reads hoisted above it (the compiler fence keeps memory
    // operations in place, the scheduling barrier everything else)
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
  }
#pragma unroll
  for (int j = 0; j < NR; ++j) acc[j] = wave_sum(acc[j]);
  if (lane == 0 && active) {
    if constexpr (GLU) {
      y[n0] = swiglu_f32(acc[0] * scale, acc[1] * scale);
    } else {
      y[n0] = acc[0] * scale;
    }
  }
}

// acc[m][j] = sum_k rows[j][k] * xs_m[k] for MX staged activation rows (row m
// at xs + m * pitch), folded across the wave: the weight pieces are loaded and
// converted once and used for every activation row. Each (m, j) sum runs over
// the pieces, then the 4-float LDS groups, in the order dot_rows_lds uses, so
// row m's result equals the single-row kernel's bit for bit.
template <typename WT, int VEC, int NR, int U, int MX>
__device__ __forceinline__ void dot_rows_lds_multi(const WT* const (&rows)[NR], const float* xs,
                                                   int pitch, long long K, int npieces, int lane,
                                                   float (&acc)[MX][NR]) {
  using V = typename RawVec<WT, VEC>::type;
  using F4 = typename RawVec<float, 4>::type;
  constexpr int PIECE = 64 * VEC;
#pragma unroll
  for (int m = 0; m < MX; ++m)
#pragma unroll
    for (int j = 0; j < NR; ++j) acc[m][j] = 0.0f;
  for (int p0 = 0; p0 < npieces; p0 += U) {
    V cur[U][NR];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const long long k = static_cast<long long>(p0 + u) * PIECE + lane * VEC;
      const bool ok = k < K;
#pragma unroll
      for (int j = 0; j < NR; ++j) {
        cur[u][j] = ok ? __builtin_nontemporal_load(reinterpret_cast<const V*>(rows[j] + k)) : V{};
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (p0 + u >= npieces) break;  // wave-uniform
#pragma unroll
      for (int h = 0; h < VEC / 4; ++h) {
        F4 a[MX];
#pragma unroll
        for (int m = 0; m < MX; ++m)
          a[m] = *reinterpret_cast<const F4*>(xs + m * pitch + (p0 + u) * PIECE + lane * 4 + h * 256);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
#pragma unroll
          for (int j = 0; j < NR; ++j) {
            const float w = static_cast<float>(cur[u][j][h * 4 + e]);
#pragma unroll
            for (int m = 0; m < MX; ++m) acc[m][j] = fmaf(a[m][e], w, acc[m][j]);
          }
        }
      }
    }
  }
#pragma unroll
  for (int m = 0; m < MX; ++m)
#pragma unroll
    for (int j = 0; j < NR; ++j) acc[m][j] = wave_sum(acc[m][j]);
}

// Output-major GEMV over MX activation rows at once (small-batch decode):
// y[m][n] = s_m * sum_k W[n][k] * x[m][k] * g[k] for m < MX, x and y
// row-major with row pitches K and N. Each workgroup stages the MX rows of
// x * gamma in LDS (MX x round_up(K, 64 * VEC) floats, sized by the caller)
// with their sums of squares, then its waves stream weight rows against all
// of them -- one pass over W serves MX outputs per row -- taking blocks of
// WAVES x R rows in turn (block b, b + gridDim.x, ...), so the staging, MX times a
// single row's, is paid once per resident workgroup rather than once per
// block. Per row the arithmetic is gemv_rows_lds_kernel's (same staging, same
// order), so each y[m] equals a single-row call on x[m] bit for bit. Same
// requirements as gemv_rows_lds_kernel.
template <typename WT, int VEC, int R, int U, int MX, bool RMS, int WAVES = 4>
__global__ __launch_bounds__(WAVES * 64) void gemv_rows_lds_multi_kernel(const WT* __restrict__ W,
                                                                  const float* __restrict__ x,
                                                                  const float* __restrict__ gamma,
                                                                  float* __restrict__ y,
                                                                  long long N, long long K,
                                                                  float eps) {
  static_assert(VEC == 4 || VEC == 8, "16-byte weight loads");
  static_assert(MX >= 2 && MX <= 4, "2 to 4 activation rows");
  constexpr int PIECE = 64 * VEC;
  extern __shared__ float xs[];
  __shared__ float wave_ss[MX][kStageWaves];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int npieces = static_cast<int>((K + PIECE - 1) / PIECE);
  const int pitch = npieces * PIECE;

  float total_ss[MX];
  stage_xs_rows<VEC, RMS, WAVES * 64, MX>(x, gamma, K, npieces, xs, pitch, &wave_ss[0][0],
                                          total_ss);
  float scale[MX];
#pragma unroll
  for (int m = 0; m < MX; ++m) scale[m] = RMS ? rms_scale(total_ss[m], K, eps) : 1.0f;

  const long long step = static_cast<long long>(gridDim.x) * WAVES * R;
  for (long long n0 = (static_cast<long long>(blockIdx.x) * WAVES + wave) * R; n0 < N; n0 += step) {
    const WT* rows[R];
#pragma unroll
    for (int r = 0; r < R; ++r) rows[r] = W + (n0 + r < N ? n0 + r : n0) * K;
    float acc[MX][R];
    dot_rows_lds_multi<WT, VEC, R, U, MX>(rows, xs, pitch, K, npieces, lane, acc);
    if (lane == 0) {
#pragma unroll
      for (int m = 0; m < MX; ++m) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
          if (n0 + r < N) y[m * N + n0 + r] = RMS ? acc[m][r] * scale[m] : acc[m][r];
        }
      }
    }
  }
}

// Fused RMSNorm + gate / up projections + SwiGLU for decode (M = 1),
// output-major weights Wg, Wu [N x K]:
//   act[n] = SiLU(s * Wg[n] . xs) * (s * Wu[n] . xs),  xs = x * gamma.
// The staged vector is shared by both projections; each wave streams the
// gate and up rows of its R outputs together (2R weight streams), so the
// intermediate gate / up vectors never reach memory and the FFN saves a
// launch. Workgroups of WAVES waves, as in gemv_rows_lds_kernel. Same
// requirements as gemv_rows_lds_kernel.
template <typename WT, int VEC, int R, int U, bool RMS, int WAVES = 4, int NP = 0, int KT = 0,
          int CH = 0>
__global__ __launch_bounds__(WAVES * 64) void gemv_rows_glu_kernel(const WT* __restrict__ Wg,
                                                            const WT* __restrict__ Wu,
                                                            const float* __restrict__ x,
                                                            const float* __restrict__ gamma,
                                                            float* __restrict__ act, long long N,
                                                            long long K, float eps) {
  static_assert(VEC == 4 || VEC == 8, "16-byte weight loads");
  constexpr int PIECE = 64 * VEC;
  extern __shared__ float xs[];
  __shared__ float wave_ss[kStageWaves];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const long long n0 = (static_cast<long long>(blockIdx.x) * WAVES + wave) * R;
  const int npieces = NP > 0 ? NP : static_cast<int>((K + PIECE - 1) / PIECE);

  float total_ss = 0.0f;
  stage_xs<VEC, RMS, WAVES * 64>(x, gamma, K, npieces, xs, wave_ss, &total_ss);
  if (n0 >= N) return;

  const WT* rows[2 * R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const long long n = n0 + r < N ? n0 + r : n0;
    rows[r] = Wg + n * K;
    rows[R + r] = Wu + n * K;
  }
  float acc[2 * R];
  if constexpr (NP > 0) {
    dot_rows_lds_fixed<WT, VEC, 2 * R, NP, KT, CH>(rows, xs, lane, acc);
  } else {
    dot_rows_lds<WT, VEC, 2 * R, U>(rows, xs, K, npieces, lane, acc);
  }
  if (lane == 0) {
    const float scale = RMS ? rms_scale(total_ss, K, eps) : 1.0f;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      if (n0 + r < N) act[n0 + r] = swiglu_f32(acc[r] * scale, acc[R + r] * scale);
    }
  }
}

// Small-batch form of gemv_rows_glu_kernel: MX activation rows (x pitch K,
// act pitch N) share each pass over Wg and Wu. The rows are staged once per
// workgroup and the workgroups (one round of residents) loop over blocks of
// WAVES outputs, as in gemv_rows_lds_multi_kernel; each wave streams one
// output's gate and up rows. Per row the arithmetic is the single-row fused
// kernel's, so act[m] equals an M = 1 call bit for bit.
template <typename WT, int VEC, int U, int MX, bool RMS, int WAVES = 4>
__global__ __launch_bounds__(WAVES * 64) void gemv_rows_glu_multi_kernel(
    const WT* __restrict__ Wg, const WT* __restrict__ Wu, const float* __restrict__ x,
    const float* __restrict__ gamma, float* __restrict__ act, long long N, long long K,
    float eps) {
  static_assert(VEC == 4 || VEC == 8, "16-byte weight loads");
  static_assert(MX >= 2 && MX <= 4, "2 to 4 activation rows");
  constexpr int PIECE = 64 * VEC;
  extern __shared__ float xs[];
  __shared__ float wave_ss[MX][kStageWaves];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int npieces = static_cast<int>((K + PIECE - 1) / PIECE);
  const int pitch = npieces * PIECE;

  float total_ss[MX];
  stage_xs_rows<VEC, RMS, WAVES * 64, MX>(x, gamma, K, npieces, xs, pitch, &wave_ss[0][0],
                                          total_ss);
  float scale[MX];
#pragma unroll
  for (int m = 0; m < MX; ++m) scale[m] = RMS ? rms_scale(total_ss[m], K, eps) : 1.0f;

  const long long step = static_cast<long long>(gridDim.x) * WAVES;
  for (long long n = static_cast<long long>(blockIdx.x) * WAVES + wave; n < N; n += step) {
    const WT* rows[2] = {Wg + n * K, Wu + n * K};
    float acc[MX][2];
    dot_rows_lds_multi<WT, VEC, 2, U, MX>(rows, xs, pitch, K, npieces, lane, acc);
    if (lane == 0) {
#pragma unroll
      for (int m = 0; m < MX; ++m) act[m * N + n] = swiglu_f32(acc[m][0] * scale[m], acc[m][1] * scale[m]);
    }
  }
}

}  // namespace gemv
}  // namespace eng
