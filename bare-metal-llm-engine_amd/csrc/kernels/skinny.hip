// skinny.hip -- linear layers over a few activation rows (5 <= M <= 64) on
// FP32 MFMA, streaming the weights once.
//
// Y[M x N] = X'[M x K] . W with X' = X (matmul) or X * gamma (rmsnorm_linear,
// whose row scale s_m = 1/sqrt(mean_k X[m][k]^2 + eps) is applied after the
// sum), W fp16 or fp32, in the reference layout [K x N] (Y = X . W) or
// output-major [N x K] (Y = X . W^T). The reference runs every M > 1 through
// its register-tiled GEMM (kernels/rmsnorm_linear.cu:195-199,
// kernels/matmul_register_tiled.cu:176-199); at a few rows a GEMM pads M to
// its tile and leaves most CUs idle (the MFMA GEMM here: ~114 us at
// 11008 x 4096 for any M <= 64 against ~15 us to read W once).
//
// v_mfma_f32_16x16x4_f32 (A[i][k] lane i + 16 k, B[k][j] lane j + 16 k,
// D[i][j] lane j + 16 (i / 4) element i % 4) with the weights loaded straight
// from HBM into the operand registers -- no LDS staging, every weight element
// passes through exactly one lane once:
//   * lane (j = l % 16, s = l / 16); the dot products run over k in a
//     lane-friendly order: k-group g (32 values of k) gives slot s the 8
//     consecutive k = g + 8 s + t, t = 0..7, at MFMA step t (a sum over k
//     does not care which slot takes which k);
//   * reference layout: lane (j, s) reads W row g + 8 s + t at columns
//     n0 + 4 j .. 4 j + 3 (16 lanes = 128 contiguous bytes of a row for
//     fp16), and column element e feeds MFMA block e as the B operand: block
//     e's column j is physical column n0 + 4 j + e, so 4 blocks cover a tile
//     of 64 columns. X is the A operand (rows m).
//   * output-major layout: lane (j, s) reads row n0 + 16 b + j of W at
//     k = g + 8 s .. + 7 (element t feeds step t) as the A operand of block
//     b; X^T is the B operand. 4 blocks b cover 64 rows of W.
//   * the X fragment is the same in both: lane (j, s) holds X[m0 + j][g + 8 s
//     + t] for t = 0..7 (two 16-byte loads from L2 per m-block; X is at most
//     64 x K floats and stays cached), times gamma[k].
//
// Work split (stream-K): the work is tiles of 64 columns of Y times units of
// 128 values of k (one k-group per wave); a grid of exactly P = 2 workgroups
// per CU (one round) takes equal runs of consecutive units, tile by tile, so
// every CU streams the same number of weight bytes whatever N is (N = 11008
// is 172 tiles: no whole number of tiles or K chunks per CU). A workgroup's 4
// waves take the k-groups of each unit in turn and their accumulators are
// summed through LDS in wave order. A tile a workgroup covers whole is
// written to Y directly (scaled by its rows' RMS factors); a tile split
// between workgroups gets one record of partial sums (and sums of squares)
// per workgroup, added by skinny_reduce_kernel in workgroup order. The split
// points depend on N, K and the CU count only -- never on M -- and each
// output's arithmetic involves only its own row of X, so a row's result is
// the same bits whichever M (5..64) it is computed in.
#include "launch.hpp"

#include <algorithm>
#include <cstddef>
#include <memory>
#include <string>
#include <type_traits>

namespace eng {
namespace {

typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef _Float16 halfx8 __attribute__((ext_vector_type(8)));
typedef _Float16 halfx4 __attribute__((ext_vector_type(4)));

constexpr int kGroup = 32;  // k values per k-group
constexpr int kWaves = 4;   // waves per workgroup (part of the summation order)
constexpr int kNB = 4;      // MFMA blocks of 16 columns per tile
constexpr int kCols = 16 * kNB;
constexpr long long kUnitK = static_cast<long long>(kGroup) * kWaves;  // k per unit
constexpr int kRS = kCols + 4;  // LDS row stride of the wave-sum tiles (floats)

// One weight register set: E consecutive elements (E = 8 or 4) of a row,
// converted to fp32 at use.
template <typename WT, int E>
struct WRaw;
template <>
struct WRaw<_Float16, 8> {
  halfx8 v;
  __device__ float at(int e) const { return static_cast<float>(v[e]); }
};
template <>
struct WRaw<_Float16, 4> {
  halfx4 v;
  __device__ float at(int e) const { return static_cast<float>(v[e]); }
};
template <>
struct WRaw<float, 8> {
  floatx4 a, b;
  __device__ float at(int e) const { return e < 4 ? a[e] : b[e - 4]; }
};
template <>
struct WRaw<float, 4> {
  floatx4 a;
  __device__ float at(int e) const { return a[e]; }
};

// E elements at p (one 16-byte load, or 8 bytes for 4 halves, or two 16-byte
// loads for 8 floats); ok false loads nothing and leaves zeros.
template <typename WT, int E>
__device__ __forceinline__ void load_raw(const WT* p, bool ok, WRaw<WT, E>& r) {
  if constexpr (std::is_same<WT, _Float16>::value && E == 8) {
    r.v = ok ? __builtin_nontemporal_load(reinterpret_cast<const halfx8*>(p)) : halfx8{};
  } else if constexpr (std::is_same<WT, _Float16>::value) {
    r.v = ok ? __builtin_nontemporal_load(reinterpret_cast<const halfx4*>(p)) : halfx4{};
  } else if constexpr (E == 8) {
    r.a = ok ? __builtin_nontemporal_load(reinterpret_cast<const floatx4*>(p)) : floatx4{};
    r.b = ok ? __builtin_nontemporal_load(reinterpret_cast<const floatx4*>(p + 4)) : floatx4{};
  } else {
    r.a = ok ? __builtin_nontemporal_load(reinterpret_cast<const floatx4*>(p)) : floatx4{};
  }
}

// The stream-K plan: U = tiles x units per tile, P workgroups, workgroup w
// taking units [w U / P, (w + 1) U / P).
struct Plan {
  long long tiles = 0;  // 64-column tiles of Y
  long long upt = 0;    // units (128 values of k) per tile
  long long U = 0;      // tiles * upt
  long long P = 0;      // workgroups
};

__host__ __device__ inline long long unit_begin(long long w, long long U, long long P) {
  return w * U / P;
}

// Workgroup whose run contains unit u.
__host__ __device__ inline long long worker_of(long long u, long long U, long long P) {
  long long w = (u * P + P - 1) / U;
  if (w >= P) w = P - 1;
  while (w + 1 < P && unit_begin(w + 1, U, P) <= u) ++w;
  while (w > 0 && unit_begin(w, U, P) > u) --w;
  return w;
}

Plan make_plan(long long N, long long K, long long cus) {
  Plan p;
  p.tiles = (N + kCols - 1) / kCols;
  p.upt = (K + kUnitK - 1) / kUnitK;
  p.U = p.tiles * p.upt;
  p.P = std::max<long long>(1, std::min<long long>(2 * cus, p.U));
  return p;
}

// MB m-blocks of 16 rows (M <= 16 MB). NK: W output-major [N x K]. RMS: X is
// multiplied by gamma (if given) and the sums of squares are produced.
// rec: [P][2][M][64] partial sums of the (at most two) tiles a workgroup
// shares with others -- slot 0 its first tile, slot 1 its last --, rec_ss
// [P][2][M] their sums of squares.
template <typename WT, bool NK, int MB, bool RMS>
__global__ __launch_bounds__(kWaves * 64, 2) void skinny_mfma_kernel(
    const WT* __restrict__ W, const float* __restrict__ x, const float* __restrict__ gamma,
    float* __restrict__ y, int M, long long N, long long K, Plan plan,
    float* __restrict__ rec, float* __restrict__ rec_ss, float eps) {
  constexpr int WAVES = kWaves;
  constexpr int NB = kNB;
  constexpr int NSET = NK ? NB : 8;  // weight register sets per k-group
  constexpr int E = NK ? 8 : NB;     // elements per set
  __shared__ float red[WAVES][16 * kRS];
  __shared__ float red_ss[WAVES][4][16 * MB];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int j = lane & 15;
  const int s = lane >> 4;
  const int tid = threadIdx.x;
  const long long w_id = blockIdx.x;
  const long long u0 = unit_begin(w_id, plan.U, plan.P);
  const long long u1 = unit_begin(w_id + 1, plan.U, plan.P);
  if (u0 >= u1) return;  // (only when U < P, which the host avoids)

  // Rows of X this lane reads (rows past M read row M - 1; never stored).
  const float* xrow[MB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    const int m = 16 * mb + j < M ? 16 * mb + j : M - 1;
    xrow[mb] = x + static_cast<long long>(m) * K;
  }
  // Without a gain the gamma loads read x instead (in bounds) and are
  // replaced by ones: no branch around a load in the steady state (a branch
  // there makes the compiler wait for every load in flight).
  const float* gsrc = (RMS && gamma != nullptr) ? gamma : x;
  const bool unit_gain = !(RMS && gamma != nullptr);

  const long long t_first = u0 / plan.upt;
  const long long t_last = (u1 - 1) / plan.upt;
  for (long long tile = t_first; tile <= t_last; ++tile) {
    const long long ua = u0 > tile * plan.upt ? u0 : tile * plan.upt;
    const long long ub = u1 < (tile + 1) * plan.upt ? u1 : (tile + 1) * plan.upt;
    const bool whole = ua == tile * plan.upt && ub == (tile + 1) * plan.upt;
    const long long k_begin = (ua - tile * plan.upt) * kUnitK;
    const long long k_next = (ub - tile * plan.upt) * kUnitK;
    const long long k_end = k_next < K ? k_next : K;
    const long long n0 = tile * kCols;

    // Weight bases: reference layout, columns n0 + 4 j .. + 3 (a 16-byte
    // piece of 4 fp32 or an 8-byte piece of 4 halves, inside N or past it:
    // N is a multiple of the 16-byte vector); a piece past N reads the row's
    // last piece instead (in bounds; it feeds only columns never stored).
    // Output-major, rows n0 + 16 b + j (rows past N read row N - 1).
    const WT* wrow[NK ? NB : 1];
    if constexpr (NK) {
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        const long long n = n0 + 16 * b + j < N ? n0 + 16 * b + j : N - 1;
        wrow[b] = W + n * K;
      }
    } else {
      const long long col = n0 + static_cast<long long>(NB) * j;
      wrow[0] = W + (col < N ? col : N - NB);
    }

    floatx4 acc[NB][MB];
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) acc[b][mb] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
    float ss[MB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) ss[mb] = 0.0f;

    // Weight register set xi of the k-group at g: reference layout, row
    // g + 8 s + xi at the lane's 4 columns; output-major, row block xi at
    // k = g + 8 s. MASKED (only the partial k-group that ends at K, K % 8 ==
    // 0): lanes whose 8 values of k lie past K load zeros.
    auto load_w = [&](WRaw<WT, E> (&w)[NSET], int xi, long long g, bool masked) {
      const long long k = g + 8 * s;
      const bool kok = !masked || k < k_end;
      if constexpr (NK) {
        load_raw<WT, E>(wrow[xi] + k, kok, w[xi]);
      } else {
        load_raw<WT, E>(wrow[0] + (k + xi) * N, kok, w[xi]);
      }
    };
    auto load_x = [&](floatx4 (&xa)[MB][2], floatx4 (&gv)[2], long long g, bool masked) {
      const long long k = g + 8 * s;
      const bool kok = !masked || k < k_end;
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        xa[mb][0] = kok ? *reinterpret_cast<const floatx4*>(xrow[mb] + k) : floatx4{};
        xa[mb][1] = kok ? *reinterpret_cast<const floatx4*>(xrow[mb] + k + 4) : floatx4{};
      }
      if constexpr (RMS) {
        gv[0] = kok ? *reinterpret_cast<const floatx4*>(gsrc + k) : floatx4{};
        gv[1] = kok ? *reinterpret_cast<const floatx4*>(gsrc + k + 4) : floatx4{};
      }
    };
    // The 8 NB MB MFMAs of one k-group held in w. Each weight register set
    // is reloaded, right after its last use, for the k-group at gr (when
    // `reload`; two k-groups ahead): reference layout, step t's row after
    // step t; output-major, row blocks two at a time after their 8 steps
    // (two accumulators interleaved so consecutive MFMAs are independent).
    // Scheduling barriers keep the reloads where they are (the scheduler
    // would sink them below the remaining MFMAs, and the next group would
    // wait for all of them at once).
    auto compute = [&](WRaw<WT, E> (&w)[NSET], const floatx4 (&xa)[MB][2],
                       const floatx4 (&gv)[2], bool reload, long long gr) {
      float xv[MB][8];
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
#pragma unroll
        for (int t = 0; t < 8; ++t) {
          const float v = xa[mb][t >> 2][t & 3];
          if constexpr (RMS) {
            ss[mb] = fmaf(v, v, ss[mb]);
            xv[mb][t] = unit_gain ? v : v * gv[t >> 2][t & 3];
          } else {
            xv[mb][t] = v;
          }
        }
      }
      if constexpr (NK) {
#pragma unroll
        for (int bp = 0; bp < NB; bp += 2) {
#pragma unroll
          for (int t = 0; t < 8; ++t) {
#pragma unroll
            for (int b = bp; b < bp + 2; ++b) {
              const float wv = w[b].at(t);
#pragma unroll
              for (int mb = 0; mb < MB; ++mb)
                acc[b][mb] = __builtin_amdgcn_mfma_f32_16x16x4f32(wv, xv[mb][t], acc[b][mb], 0, 0, 0);
            }
          }
          if (reload) {
            load_w(w, bp, gr, false);
            load_w(w, bp + 1, gr, false);
          }
          __builtin_amdgcn_sched_barrier(0);
        }
      } else {
#pragma unroll
        for (int t = 0; t < 8; ++t) {
#pragma unroll
          for (int b = 0; b < NB; ++b) {
            const float wv = w[t].at(b);
#pragma unroll
            for (int mb = 0; mb < MB; ++mb)
              acc[b][mb] = __builtin_amdgcn_mfma_f32_16x16x4f32(xv[mb][t], wv, acc[b][mb], 0, 0, 0);
          }
          if (reload) load_w(w, t, gr, false);
          __builtin_amdgcn_sched_barrier(0);
        }
      }
    };

    // Whole k-groups of the range, wave w taking g = k_begin + 32 (w + WAVES
    // i), software-pipelined: weights two k-groups ahead in two register sets
    // (wa: the wave's groups 0, 2, 4, ...; wb: 1, 3, 5, ...), each set
    // reloaded as it is consumed, X one k-group ahead. The steady-state loop
    // is straight-line code (every reload target exists); the last two or
    // three groups follow it, then at most one partial group (the range that
    // ends at K, when K % 32 != 0).
    const long long full_end = k_begin + (k_end - k_begin) / kGroup * kGroup;
    const long long step = static_cast<long long>(WAVES) * kGroup;
    long long g = k_begin + static_cast<long long>(wave) * kGroup;
    const long long nfull = g < full_end ? (full_end - g + step - 1) / step : 0;
    WRaw<WT, E> wa[NSET], wb[NSET];
    floatx4 xa0[MB][2], xa1[MB][2], gv0[2], gv1[2];
    if (nfull > 0) {
      // wb's first group (the same group again when the wave has only one:
      // an unconditional load keeps the loop's count of outstanding loads
      // exact)
      const long long gb = nfull > 1 ? g + step : g;
#pragma unroll
      for (int xi = 0; xi < NSET; ++xi) load_w(wa, xi, g, false);
      load_x(xa0, gv0, g, false);
#pragma unroll
      for (int xi = 0; xi < NSET; ++xi) load_w(wb, xi, gb, false);
    }
    long long i = 0;
    for (; i + 3 < nfull; i += 2) {
      load_x(xa1, gv1, g + step, false);
      __builtin_amdgcn_sched_barrier(0);
      compute(wa, xa0, gv0, true, g + 2 * step);
      load_x(xa0, gv0, g + 2 * step, false);
      __builtin_amdgcn_sched_barrier(0);
      compute(wb, xa1, gv1, true, g + 3 * step);
      g += 2 * step;
    }
    if (i < nfull) {
      const bool more1 = i + 1 < nfull;
      const bool more2 = i + 2 < nfull;
      if (more1) load_x(xa1, gv1, g + step, false);
      compute(wa, xa0, gv0, more2, g + 2 * step);
      if (more1) {
        if (more2) load_x(xa0, gv0, g + 2 * step, false);
        compute(wb, xa1, gv1, false, 0);
        if (more2) compute(wa, xa0, gv0, false, 0);
      }
    }
    if (full_end < k_end && ((full_end - k_begin) / kGroup) % WAVES == wave) {
#pragma unroll
      for (int xi = 0; xi < NSET; ++xi) load_w(wa, xi, full_end, true);
      load_x(xa0, gv0, full_end, true);
      compute(wa, xa0, gv0, false, 0);
    }

    // Sums of squares: lane (j, s) holds row 16 mb + j over slot s's k.
    if constexpr (RMS) {
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) red_ss[wave][s][16 * mb + j] = ss[mb];
    }
    // Wave sums through LDS, one m-block at a time: each wave stores its
    // 16 x 64 tile, then the workgroup adds the WAVES tiles in wave order.
    const int slot = tile == t_first ? 0 : 1;
    float* rec_tile = rec + (w_id * 2 + slot) * static_cast<long long>(M) * kCols;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      __syncthreads();  // the previous tile's (or m-block's) sums have been read
#pragma unroll
      for (int b = 0; b < NB; ++b) {
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          int r, c;
          if constexpr (NK) {
            r = j;                   // m = 16 mb + j
            c = 16 * b + 4 * s + v;  // n = n0 + c
          } else {
            r = 4 * s + v;           // m = 16 mb + r
            c = NB * j + b;          // n = n0 + c
          }
          red[wave][r * kRS + c] = acc[b][mb][v];
        }
      }
      __syncthreads();
      for (int idx = tid; idx < 16 * kCols; idx += WAVES * 64) {
        const int r = idx / kCols;
        const int c = idx - r * kCols;
        const int m = 16 * mb + r;
        if (m >= M) continue;
        float v = red[0][r * kRS + c];
#pragma unroll
        for (int w2 = 1; w2 < WAVES; ++w2) v += red[w2][r * kRS + c];
        if (whole) {
          const long long n = n0 + c;
          if (n >= N) continue;
          if constexpr (RMS) {
            float tot = 0.0f;
#pragma unroll
            for (int w2 = 0; w2 < WAVES; ++w2)
#pragma unroll
              for (int q = 0; q < 4; ++q) tot += red_ss[w2][q][m];
            v *= 1.0f / sqrtf(tot / static_cast<float>(K) + eps);
          }
          y[static_cast<long long>(m) * N + n] = v;
        } else {
          rec_tile[static_cast<long long>(m) * kCols + c] = v;
        }
      }
    }
    if (RMS && !whole) {
      for (int m = tid; m < M; m += WAVES * 64) {
        float tot = 0.0f;
#pragma unroll
        for (int w2 = 0; w2 < WAVES; ++w2)
#pragma unroll
          for (int q = 0; q < 4; ++q) tot += red_ss[w2][q][m];
        rec_ss[(w_id * 2 + slot) * M + m] = tot;
      }
    }
    __syncthreads();  // red / red_ss are reused by the next tile
  }
}

// Tiles split between workgroups: y[m][n] = s_m * sum over the tile's
// workgroups, in workgroup order, of their records (s_m = 1 without RMS;
// with RMS from the records' sums of squares, added in the same order).
// Row m is blockIdx.y; columns of tiles that one workgroup covered whole are
// skipped (already written). Up to 4 records' loads in flight per batch.
template <bool RMS>
__global__ __launch_bounds__(256) void skinny_reduce_kernel(const float* __restrict__ rec,
                                                            const float* __restrict__ rec_ss,
                                                            float* __restrict__ y, int M,
                                                            long long N, long long K, Plan plan,
                                                            float eps) {
  const long long n = static_cast<long long>(blockIdx.x) * 256 + threadIdx.x;
  const int m = blockIdx.y;
  if (n >= N) return;
  const long long tile = n / kCols;
  const int c = static_cast<int>(n - tile * kCols);
  const long long wf = worker_of(tile * plan.upt, plan.U, plan.P);
  const long long wl = worker_of(tile * plan.upt + plan.upt - 1, plan.U, plan.P);
  if (wf == wl) return;  // one workgroup covered the tile: written directly
  float v = 0.0f;
  float tot = 0.0f;
  for (long long w0 = wf; w0 <= wl; w0 += 4) {
    float p[4], q[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const long long w = w0 + i <= wl ? w0 + i : wl;
      const int slot = unit_begin(w, plan.U, plan.P) / plan.upt == tile ? 0 : 1;
      const long long r = w * 2 + slot;
      p[i] = rec[(r * M + m) * kCols + c];
      if constexpr (RMS) q[i] = rec_ss[r * M + m];
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v += w0 + i <= wl ? p[i] : 0.0f;
      if constexpr (RMS) tot += w0 + i <= wl ? q[i] : 0.0f;
    }
  }
  if constexpr (RMS) v *= 1.0f / sqrtf(tot / static_cast<float>(K) + eps);
  y[static_cast<long long>(m) * N + n] = v;
}

std::size_t scratch_for(const Plan& p, long long M) {
  return static_cast<std::size_t>(p.P) * 2 * M * (kCols + 1) * sizeof(float);
}

template <typename WT, bool NK, int MB, bool RMS>
void run_skinny(const SkinnyArgs& a, hipStream_t stream) {
  const long long N = a.N;
  const long long K = a.K;
  const int M = static_cast<int>(a.M);
  const Plan plan = make_plan(N, K, device_cu_count());
  ENG_CHECK(plan.P <= 0x7fffffffLL, "linear: grid too large for one launch");
  const std::size_t need = scratch_for(plan, M);
  float* rec = nullptr;
  std::unique_ptr<StreamScratch> ws;
  if (a.scratch != nullptr) {
    ENG_CHECK(need <= a.scratch_bytes,
              "linear: the few-row kernel's partial sums need " + std::to_string(need) +
                  " bytes of scratch, more than the " + std::to_string(a.scratch_bytes) +
                  " bytes provided");
    rec = static_cast<float*>(a.scratch);
  } else {
    ws = std::make_unique<StreamScratch>(stream, need);
    rec = static_cast<float*>(ws->get());
  }
  float* rec_ss = rec + plan.P * 2 * static_cast<long long>(M) * kCols;
  skinny_mfma_kernel<WT, NK, MB, RMS><<<static_cast<unsigned>(plan.P), kWaves * 64, 0, stream>>>(
      static_cast<const WT*>(a.W), a.x, a.gamma, a.y, M, N, K, plan, rec, rec_ss, a.eps);
  ENG_LAUNCH_CHECK();
  // Every workgroup takes whole tiles: nothing left to add.
  if (plan.U % plan.P == 0 && (plan.U / plan.P) % plan.upt == 0) return;
  skinny_reduce_kernel<RMS><<<dim3(static_cast<unsigned>((N + 255) / 256), M), 256, 0, stream>>>(
      rec, rec_ss, a.y, M, N, K, plan, a.eps);
  ENG_LAUNCH_CHECK();
}

template <typename WT, bool NK, bool RMS>
void dispatch_mb(const SkinnyArgs& a, hipStream_t stream) {
  switch ((a.M + 15) / 16) {
    case 1: run_skinny<WT, NK, 1, RMS>(a, stream); break;
    case 2: run_skinny<WT, NK, 2, RMS>(a, stream); break;
    case 3: run_skinny<WT, NK, 3, RMS>(a, stream); break;
    default: run_skinny<WT, NK, 4, RMS>(a, stream); break;
  }
}

template <typename WT, bool NK>
void dispatch_rms(const SkinnyArgs& a, hipStream_t stream) {
  if (a.rms) {
    dispatch_mb<WT, NK, true>(a, stream);
  } else {
    dispatch_mb<WT, NK, false>(a, stream);
  }
}

}  // namespace

bool skinny_applies(const SkinnyArgs& a) {
  if (a.M < kSkinnyMinRows || a.M > kSkinnyMaxRows) return false;
  const long long vpw = a.w == Elem::F16 ? 8 : 4;
  if (a.K % 8 != 0) return false;
  if (!a.w_nk && a.N % vpw != 0) return false;
  return aligned_to(a.W, 16) && aligned_to(a.x, 16) &&
         (a.gamma == nullptr || aligned_to(a.gamma, 16));
}

std::size_t skinny_scratch_bytes(const SkinnyArgs& a) {
  return scratch_for(make_plan(a.N, a.K, device_cu_count()), a.M);
}

void launch_skinny(const SkinnyArgs& a, hipStream_t stream) {
  ENG_CHECK(skinny_applies(a), "linear: shape not supported by the few-row kernel");
  if (a.w == Elem::F16) {
    if (a.w_nk) {
      dispatch_rms<_Float16, true>(a, stream);
    } else {
      dispatch_rms<_Float16, false>(a, stream);
    }
  } else {
    if (a.w_nk) {
      dispatch_rms<float, true>(a, stream);
    } else {
      dispatch_rms<float, false>(a, stream);
    }
  }
}

}  // namespace eng
