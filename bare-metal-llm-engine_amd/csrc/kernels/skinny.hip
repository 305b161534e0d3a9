// skinny.hip -- linear layers over a few activation rows (5 <= M <= 64; fp16
// weights up to 32, past that the fp16-MFMA GEMM) on the matrix cores,
// streaming the weights once.
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
// Work split (stream-K), shared by both layouts: the work is tiles of 64
// weight rows (output-major) or columns (reference layout) times units of
// 128 values of k; a grid of exactly P = 2 workgroups per CU (one round)
// takes equal runs of consecutive units, tile by tile, so every CU streams
// the same number of weight bytes whatever N is (N = 11008 is 172 tiles: no
// whole number of tiles or K chunks per CU). A tile a workgroup covers whole
// is written to Y directly (scaled by its rows' RMS factors); a tile split
// between workgroups gets one record of partial sums (and sums of squares)
// per workgroup, added by skinny_reduce_kernel in workgroup order. The split
// points depend on N, K and the CU count only -- never on M -- and each
// output's arithmetic involves only its own row of X, so a row's result is
// the same bits whichever M (5..64; fp16 W 5..32) it is computed in.
//
// skinny_nk_kernel covers a unit the same way for output-major W (its
// weights straight into registers, or at one m-block of fp16 W through LDS
// stages) and for reference-layout fp16 W (through LDS stages, read
// transposed); skinny_mfma_kernel takes reference-layout fp32 W. At 11008 x
// 4096 fp16 W [K x N] the staged form took 25.5 us at M = 16 (27.6 with the
// third activation term) against 31.1 us for skinny_mfma_kernel (fp32 MFMA on
// converted weights).
#include "device_sync.hpp"
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

// Maximum over each group of 32 consecutive lanes, in all of them: DPP
// quad_perm xor-1 and xor-2, row_half_mirror and row_mirror give each 16-lane
// row's maximum, one shuffle joins the two rows of a group. A maximum is
// exact, so any combining order gives the same bits as a shuffle tree (five
// LDS-crossbar round trips, where this takes one).
template <int CTRL>
__device__ __forceinline__ float dpp_max(float x) {
  const int y = __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xF, 0xF, false);
  return fmaxf(x, __builtin_bit_cast(float, y));
}
__device__ __forceinline__ float group32_max(float x) {
  x = dpp_max<0xB1>(x);   // quad_perm [1, 0, 3, 2]
  x = dpp_max<0x4E>(x);   // quad_perm [2, 3, 0, 1]
  x = dpp_max<0x141>(x);  // row_half_mirror
  x = dpp_max<0x140>(x);  // row_mirror
  return fmaxf(x, __shfl_xor(x, 16));
}

typedef short v4i16 __attribute__((ext_vector_type(4)));

// Chunk swizzle of the reference-layout weight stage: row r (one k, 64
// columns = 8 chunks of 16 bytes) keeps chunk c at position c ^ kn_swz(r).
// A transposing read touches 16 rows x 32 bytes (rows 8 s + e and 8 s + e
// + 4 for the four lane groups s, e = 0..3); an even swizzle keeps each
// 32-byte pair whole, and (s + e / 2) spreads the pairs evenly over the
// four pair positions, so no bank takes more than the minimum.
__device__ __forceinline__ int kn_swz(int r) { return (((r >> 3) + (r >> 1)) & 3) << 1; }

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

// floor(a / b) for 0 <= a < 2^53, b > 0: a double-precision estimate
// corrected with integer multiplies (a 64-bit integer division costs ~150
// instructions on the GPU; the reduce kernel needs several per thread).
__host__ __device__ inline long long floor_div(long long a, long long b) {
  long long q = static_cast<long long>(static_cast<double>(a) / static_cast<double>(b));
  while (q > 0 && q * b > a) --q;
  while ((q + 1) * b <= a) ++q;
  return q;
}

__host__ __device__ inline long long unit_begin(long long w, long long U, long long P) {
  return floor_div(w * U, P);
}

// Workgroup whose run contains unit u.
__host__ __device__ inline long long worker_of(long long u, long long U, long long P) {
  long long w = floor_div(u * P + P - 1, U);
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

// Reference layout (used with NK false; the output-major instantiation is
// superseded by skinny_nk_kernel). v_mfma_f32_16x16x4_f32 (A[i][k] lane
// i + 16 k, B[k][j] lane j + 16 k, D[i][j] lane j + 16 (i / 4) element i % 4)
// with the weights loaded straight from HBM into the operand registers:
//   * lane (j = l % 16, s = l / 16); k-group g (32 values of k) gives slot s
//     the 8 consecutive k = g + 8 s + t, t = 0..7, at MFMA step t (a sum over
//     k does not care which slot takes which k);
//   * lane (j, s) reads W row g + 8 s + t at columns n0 + 4 j .. 4 j + 3 (16
//     lanes = 128 contiguous bytes of a row for fp16), and column element e
//     feeds MFMA block e as the B operand: block e's column j is physical
//     column n0 + 4 j + e, so 4 blocks cover a tile of 64 columns. X is the A
//     operand (rows m): lane (j, s) holds X[m0 + j][g + 8 s + t] for t = 0..7
//     (two 16-byte loads from L2 per m-block), times gamma[k].
// A workgroup's 4 waves take the k-groups of each unit in turn and their
// accumulators are summed through LDS in wave order.
// MB m-blocks of 16 rows (M <= 16 MB). RMS: X is multiplied by gamma (if
// given) and the sums of squares are produced.
// rec: [P][2][M][64] partial sums of the (at most two) tiles a workgroup
// shares with others -- slot 0 its first tile, slot 1 its last --, rec_ss
// [P][2][M] their sums of squares.
template <typename WT, bool NK, int MB, bool RMS>
__global__ __launch_bounds__(kWaves * 64, MB >= 3 ? 1 : 2) void skinny_mfma_kernel(
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

template <typename WT>
struct WVec;
template <>
struct WVec<_Float16> {
  using type = halfx8;
};
template <>
struct WVec<float> {
  using type = floatx4;
};

// Output-major W [N x K]: wave w of a workgroup owns the 16 weight rows
// n0 + 16 w .. + 15 of each tile and runs the workgroup's whole range of
// units over them; the activations of a unit (16 MB rows x 128 values of k,
// times gamma) are staged in LDS once per workgroup. Lane (j, s) loads 16
// bytes of row n0 + 16 w + j at k = k_u + 4 E i + E s (E elements per 16
// bytes, i the load of the unit), so one load instruction covers 16 rows x 64
// bytes and a wave's consecutive loads continue along the same rows: each row
// is read in 256-byte runs per unit (64-byte runs spread over row blocks and
// waves streamed at 4.4-4.7 TB/s).
//
// fp16 weights: v_mfma_f32_16x16x32_f16 takes a load as it arrives (lane
// (j, s) holds A[j][8 s .. 8 s + 7] of the 32 values of k of load i). The
// activations enter as three fp16 planes: per unit and row, t = x' 2^e with
// the power of two 2^e putting max |t| in [2^14, 2^15), hi = fp16(t), lo =
// fp16((t - hi) 2^11) and lo2 = fp16(((t - hi) 2^11 - lo) 2^11) -- each
// difference is exact in fp32 and each term keeps the next 11 bits, so hi +
// lo 2^-11 + lo2 2^-22 is t exactly (every x' whose bits reach no lower than
// 2^-39 of the unit's largest) and the products hi w, lo w, lo2 w are exact
// in fp32. Three MFMAs per load and m-block (one accumulator per plane);
// after each unit the row's partial (acc_hi + (acc_lo + acc_lo2 2^-11)
// 2^-11) 2^-e is added to its running sum: the fp32 arithmetic, exact
// products and fp32 sums, in 3/8 of the matrix cycles of fp32 MFMA on the
// same data.
// fp32 weights: v_mfma_f32_16x16x4_f32, 8 MFMAs per load (step t takes
// element t, k slot s), X' in fp32 planes.
// Both: D[i][j] (lane j + 16 (i / 4), element i % 4) is weight row 16 w + i
// against activation row 16 mb + j.
//
// Units run in one software pipeline across the workgroup's tiles: each
// weight load is reissued for the next unit right after its values are
// taken (one unit of weights in flight per wave -- with this access pattern
// more in flight measured slower: 16 rows x 256 bytes per wave streams 90 MB
// in 18.2 us, two units ahead 21.6, three 22.4), the next unit's X loaded at
// the start of a unit and written to the other LDS buffer at its end; one
// barrier per unit.
// Staging: thread t takes k chunk t % 32 (4 values) of rows t / 32 + 8 r,
// whatever MB: it multiplies by gamma, adds the squares of x into its per-row
// sum of squares (RMS), and for fp16 weights takes the maximum |x'| over the
// row's 32 chunk threads (adjacent lanes, group32_max) for the scale. The tile end
// folds the sums of squares the same way -- orders fixed by the plan, never
// by M.
// LDS, per buffer: fp32 X' as 16-byte chunks, row m at m * 32, chunk c at
// c ^ (m & 7); fp16 planes with 8-value chunks, row m at m * 16, chunk c at
// c ^ (m & 15) (the 16 rows one MFMA operand read touches land in different
// banks).
template <typename WT, int MB, bool RMS, int WMODE = 0>
__global__ __launch_bounds__(kWaves * 64, 2) void skinny_nk_kernel(
    const WT* __restrict__ W, const float* __restrict__ x, const float* __restrict__ gamma,
    float* __restrict__ y, int M, long long N, long long K, Plan plan,
    float* __restrict__ rec, float* __restrict__ rec_ss, float eps) {
  using WV = typename WVec<WT>::type;
  constexpr bool H = std::is_same<WT, _Float16>::value;    // fp16 MFMA path
  // WMODE 0: output-major W into registers; 1: reference layout (KN) and 2:
  // output-major, both through LDS stages (fp16).
  constexpr bool KN = WMODE == 1;
  constexpr bool STAGED = WMODE != 0;
  static_assert(!STAGED || H, "the LDS-staged forms are fp16 only");
  constexpr int E = 16 / static_cast<int>(sizeof(WT));     // elements per 16-byte load
  constexpr int LPU = static_cast<int>(kUnitK) / (4 * E);  // loads per unit per lane
  constexpr int ROWS = 16 * MB;
  constexpr int CPR = static_cast<int>(kUnitK) / 4;        // 4-value chunks per row per unit
  constexpr int THREADS = kWaves * 64;
  constexpr int SPT = ROWS * CPR / THREADS;                // staged chunks per thread
  constexpr int HCR = static_cast<int>(kUnitK) / 8;        // 8-value chunks per fp16 plane row
  static_assert(SPT * THREADS == ROWS * CPR, "staging covers the unit");
  // One LDS buffer: fp32 X' (ROWS x 32 16-byte chunks), or the fp16 hi, lo
  // and lo2 planes (ROWS x 16 chunks each) and the rows' descale factors 2^-e.
  struct XBuf {
    floatx4 f[H ? 1 : ROWS * CPR];
    halfx8 hi[H ? ROWS * HCR : 1];
    halfx8 lo[H ? ROWS * HCR : 1];
    halfx8 lo2[H ? ROWS * HCR : 1];
    float ds[H ? ROWS : 1];
  };
  // Two X buffers where they fit beside the weight stages and the RMS sums
  // in half the LDS (two workgroups per CU), else one (staged weights, read
  // and rewritten between two barriers per unit): the reference layout at
  // 17-32 rows with the three fp16 planes.
  constexpr int XB =
      (STAGED && 2 * sizeof(XBuf) + 2 * 128 * 8 * sizeof(halfx8) + 4 * ROWS > 80 * 1024) ? 1 : 2;
  __shared__ XBuf xbuf[XB];
  __shared__ float ssc[RMS ? ROWS : 1];
  // Staged weights: two stages of a unit's 16 KiB block of W (KN: 128 rows
  // of k x 8 chunks of 16 bytes; output-major: 64 rows x 16 chunks).
  __shared__ halfx8 wst[STAGED ? 2 * 128 * 8 : 1];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int j = lane & 15;
  const int s = lane >> 4;
  const long long w_id = blockIdx.x;
  const long long u0 = unit_begin(w_id, plan.U, plan.P);
  const long long u1 = unit_begin(w_id + 1, plan.U, plan.P);
  if (u0 >= u1) return;  // (only when U < P, which the host avoids)
  const long long upt = plan.upt;
  const long long t_first = u0 / upt;

  // ---- staging ----
  // Loads past K or past the range read offset 0 of the same row and are
  // zeroed at the store (no branch around a load); without a gain the gamma
  // loads read x and are replaced by ones.
  const bool has_g = gamma != nullptr;
  const float* gsrc = has_g ? gamma : x;
  const int qc = tid % CPR;
  // One unit's X and gamma in registers, and whether its k chunk is in range.
  struct XStage {
    floatx4 xr[SPT];
    floatx4 gr;
    bool xok;
  };
  float ssr[RMS ? SPT : 1];
#pragma unroll
  for (int r = 0; r < (RMS ? SPT : 1); ++r) ssr[r] = 0.0f;
  // X of unit u, which is unit ku of its tile.
  auto load_x = [&](XStage& S, long long u, long long ku) __attribute__((always_inline)) {
    const long long k = ku * kUnitK + 4 * qc;
    S.xok = u < u1 && k < K;
    const long long ko = S.xok ? k : 0;
#pragma unroll
    for (int r = 0; r < SPT; ++r) {
      const int m = tid / CPR + (THREADS / CPR) * r;
      S.xr[r] = *reinterpret_cast<const floatx4*>(x + static_cast<long long>(m < M ? m : M - 1) * K + ko);
    }
    S.gr = *reinterpret_cast<const floatx4*>(gsrc + ko);
  };
  auto store_x = [&](const XStage& S, XBuf& xb) __attribute__((always_inline)) {
    const auto& xr = S.xr;
    const auto& gr = S.gr;
    const bool xok = S.xok;
    const floatx4 zero = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
    const floatx4 g = has_g ? gr : floatx4{1.0f, 1.0f, 1.0f, 1.0f};
#pragma unroll
    for (int r = 0; r < SPT; ++r) {
      const int m = tid / CPR + (THREADS / CPR) * r;
      const floatx4 v = xok ? xr[r] : zero;
      if constexpr (RMS) {
        ssr[r] = fmaf(v[0], v[0], ssr[r]);
        ssr[r] = fmaf(v[1], v[1], ssr[r]);
        ssr[r] = fmaf(v[2], v[2], ssr[r]);
        ssr[r] = fmaf(v[3], v[3], ssr[r]);
      }
      const floatx4 xv = v * g;
      if constexpr (H) {
        static_assert(CPR == 32, "a row's chunk threads are one 32-lane group");
        const float amax = group32_max(
            fmaxf(fmaxf(fabsf(xv[0]), fabsf(xv[1])), fmaxf(fabsf(xv[2]), fabsf(xv[3]))));
        int ex = 0;
        (void)frexpf(amax, &ex);  // amax = f 2^ex, f in [0.5, 1) (ex = 0 for 0, inf, nan)
        const int e = min(15 - ex, 126);
        halfx4 h, l, l2;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const float t = ldexpf(xv[q], e);
          h[q] = static_cast<_Float16>(t);
          const float r1 = (t - static_cast<float>(h[q])) * 2048.0f;
          l[q] = static_cast<_Float16>(r1);
          l2[q] = static_cast<_Float16>((r1 - static_cast<float>(l[q])) * 2048.0f);
        }
        const int pos = m * HCR + ((qc >> 1) ^ (m & 15));
        reinterpret_cast<halfx4*>(&xb.hi[pos])[qc & 1] = h;
        reinterpret_cast<halfx4*>(&xb.lo[pos])[qc & 1] = l;
        reinterpret_cast<halfx4*>(&xb.lo2[pos])[qc & 1] = l2;
        if (qc == 0) xb.ds[m] = ldexpf(1.0f, -e);
      } else {
        xb.f[m * CPR + (qc ^ (m & 7))] = xv;
      }
    }
  };

  // ---- weights ----
  // Cursor over the workgroup's units: unit, tile, unit within the tile, and
  // the lane's weight row.
  struct Cursor {
    long long u, tile, ku;
    const WT* row;
  };
  auto row_of = [&](long long tile) {
    long long n = tile * kCols + 16 * wave + j;
    n = n < N ? n : N - 1;
    return W + n * K;
  };
  auto advance = [&](Cursor& c) {
    ++c.u;
    if (++c.ku == upt) {
      c.ku = 0;
      ++c.tile;
      c.row = row_of(c.tile);
    }
  };
  // Load i of the cursor's unit (past K or past the range: offset 0 of the
  // row, zeroed at use or never used).
  auto w_src = [&](const Cursor& c, int i) -> const WV* {
    const long long k = c.ku * kUnitK + 4 * E * i + E * s;
    return reinterpret_cast<const WV*>(c.row + ((c.u < u1 && k < K) ? k : 0));
  };
  auto load_w = [&](WV (&w)[LPU], const Cursor& c) {
#pragma unroll
    for (int i = 0; i < LPU; ++i) w[i] = __builtin_nontemporal_load(w_src(c, i));
  };

  // acc: the running sums (fp32 path: the MFMA accumulators themselves);
  // ach, acl, acm: the fp16 path's hi, lo and lo2 accumulators of a unit.
  floatx4 acc[MB], ach[H ? MB : 1], acl[H ? MB : 1], acm[H ? MB : 1];
  auto zero4 = [] { return floatx4{0.0f, 0.0f, 0.0f, 0.0f}; };
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) acc[mb] = zero4();
  if constexpr (H) {
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) ach[mb] = acl[mb] = acm[mb] = zero4();
  }

  // The LPU loads of the unit at cur against buffer xb; load i of w is
  // reissued for the cursor `next` once its values are taken (scheduling
  // barriers keep the reload below that point, so it reuses the set's
  // registers and the loop carries no register copies, which would wait for
  // the loads in flight). Pieces past K (the last unit of a row when
  // K % 128 != 0) are zeroed here.
  auto compute = [&](WV (&w)[LPU], const XBuf& xb, const Cursor& cur, const Cursor& next)
      __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < LPU; ++i) {
      const bool kok = cur.ku * kUnitK + 4 * E * i + E * s < K;
      if constexpr (H) {
        const halfx8 wi = kok ? w[i] : halfx8{};
        halfx8 bh[MB], bl[MB], bm[MB];
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) {
          const int pos = (16 * mb + j) * HCR + ((4 * i + s) ^ (j & 15));
          bh[mb] = xb.hi[pos];
          bl[mb] = xb.lo[pos];
          bm[mb] = xb.lo2[pos];
        }
        __builtin_amdgcn_sched_barrier(0);
        w[i] = __builtin_nontemporal_load(w_src(next, i));
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) {
          ach[mb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wi, bh[mb], ach[mb], 0, 0, 0);
          acl[mb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wi, bl[mb], acl[mb], 0, 0, 0);
          acm[mb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wi, bm[mb], acm[mb], 0, 0, 0);
        }
      } else {
        const WV wi = kok ? w[i] : WV{};
        floatx4 xf[MB];
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) xf[mb] = xb.f[(16 * mb + j) * CPR + ((4 * i + s) ^ (j & 7))];
        __builtin_amdgcn_sched_barrier(0);
        w[i] = __builtin_nontemporal_load(w_src(next, i));
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int t = 0; t < 4; ++t) {
#pragma unroll
          for (int mb = 0; mb < MB; ++mb)
            acc[mb] = __builtin_amdgcn_mfma_f32_16x16x4f32(wi[t], xf[mb][t], acc[mb], 0, 0, 0);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    if constexpr (H) {
      // the unit's partial, descaled, into the running sums
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        const float d = xb.ds[16 * mb + j];
        const floatx4 p = ach[mb] + (acl[mb] + acm[mb] * (1.0f / 2048.0f)) * (1.0f / 2048.0f);
        acc[mb] += p * d;
        ach[mb] = acl[mb] = acm[mb] = zero4();
      }
    }
  };

  // KN (reference layout W [K x N], fp16): a unit's 128 x 64 block of W is
  // loaded in 16-byte pieces -- thread slot g = (4 q + wave) * 64 + lane
  // takes 16 bytes of row g / 8 (one wave load: 8 rows x 128 bytes) --
  // written to an LDS stage (chunk c of row r at position c ^ kn_swz(r)), and
  // each wave reads its A operands from there transposed: lane (j, s) of load
  // i gets column 16 wave + j at k = 32 i + 8 s + t, t = 0..7 (the same
  // fragment skinny_nk_kernel loads from an output-major row), with two gfx950
  // transposing LDS reads (ds_read_b64_tr_b16) per fragment. Rows past K read row 0 of the unit and columns past
  // N chunk 0 of the tile; both are zeroed or dropped at use. (Loading
  // straight into LDS measured no faster: the compiler then waits for those
  // loads before any LDS access it cannot prove disjoint, which serialises
  // them with the unit's arithmetic.)
  // WMODE 2 (output-major W through LDS): thread slot g takes 16 bytes (8
  // values of k) of weight row g / 16 of the tile at k chunk g % 16 (one wave
  // load: 4 rows x 256 bytes), stored at chunk position (g % 16) ^ (row % 16)
  // of the row's 256 bytes; lane (j, s) of load i reads row 16 wave + j, chunk
  // 4 i + s with one 16-byte read (the 16 rows of a lane group hit 16
  // distinct chunk positions). Rows past N read row N - 1, chunks past K the
  // row's first; zeroed or dropped at use.
  auto load_wk = [&](halfx8 (&wr)[4], const Cursor& c) __attribute__((always_inline)) {
    const long long kbase = c.ku * kUnitK;
    const long long n0 = c.tile * kCols;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int g = (4 * q + wave) * 64 + lane;
      if constexpr (KN) {
        const int r = g >> 3;
        const int cch = (g & 7) ^ kn_swz(r);
        const long long off = (kbase + r < K ? static_cast<long long>(r) * N : 0) +
                              (n0 + 8 * cch < N ? 8 * cch : 0);
        wr[q] = __builtin_nontemporal_load(reinterpret_cast<const halfx8*>(W + kbase * N + n0 + off));
      } else {
        const long long n = n0 + (g >> 4) < N ? n0 + (g >> 4) : N - 1;
        const long long k = kbase + 8 * (g & 15);
        wr[q] = __builtin_nontemporal_load(reinterpret_cast<const halfx8*>(W + n * K + (k < K ? k : 0)));
      }
    }
  };
  auto put_wk = [&](const halfx8 (&wr)[4], int st) __attribute__((always_inline)) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int g = (4 * q + wave) * 64 + lane;
      const int pos = KN ? g : (g & ~15) | ((g & 15) ^ ((g >> 4) & 15));
      wst[st * 1024 + pos] = wr[q];
    }
  };
  auto compute_kn = [&](const XBuf& xb, int st, const Cursor& cur) __attribute__((always_inline)) {
    const _Float16* ws = reinterpret_cast<const _Float16*>(&wst[st * 1024]);
#pragma unroll
    for (int i = 0; i < LPU; ++i) {
      const bool kok = cur.ku * kUnitK + 4 * E * i + E * s < K;
      halfx8 wv;
      if constexpr (KN) {
        // Two transposing reads of 4 rows each: within each 16-lane group,
        // lane L names 8 bytes (row r0 + L / 4, columns 16 wave + 4 (L % 4)
        // .. + 3) and lane j receives column 16 wave + j of the 4 rows.
        const int a4 = j & 3;
        const int c = 2 * wave + (a4 >> 1);
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int r = 32 * i + 8 * s + 4 * h + (j >> 2);
          const int off = r * 128 + ((c ^ kn_swz(r)) << 4) + ((a4 & 1) << 3);
          const halfx4 v = __builtin_bit_cast(
              halfx4, __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4i16*)(
                          (__attribute__((address_space(3))) char*)ws + off)));
#pragma unroll
          for (int e = 0; e < 4; ++e) wv[4 * h + e] = v[e];
        }
      } else {
        wv = wst[st * 1024 + (16 * wave + j) * 16 + ((4 * i + s) ^ j)];
      }
      const halfx8 wi = kok ? wv : halfx8{};
      halfx8 bh[MB], bl[MB], bm[MB];
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        const int pos = (16 * mb + j) * HCR + ((4 * i + s) ^ (j & 15));
        bh[mb] = xb.hi[pos];
        bl[mb] = xb.lo[pos];
        bm[mb] = xb.lo2[pos];
      }
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        ach[mb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wi, bh[mb], ach[mb], 0, 0, 0);
        acl[mb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wi, bl[mb], acl[mb], 0, 0, 0);
        acm[mb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wi, bm[mb], acm[mb], 0, 0, 0);
      }
    }
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      const float d = xb.ds[16 * mb + j];
      const floatx4 p = ach[mb] + (acl[mb] + acm[mb] * (1.0f / 2048.0f)) * (1.0f / 2048.0f);
      acc[mb] += p * d;
      ach[mb] = acl[mb] = acm[mb] = zero4();
    }
  };

  // Tile end: whole tiles go to y (scaled by their rows' RMS factors), split
  // tiles to this workgroup's record slot.
  auto finish = [&](const Cursor& c) __attribute__((always_inline)) {
    const long long tile = c.tile;
    const bool whole = tile * upt >= u0 && c.ku == upt - 1;
    const int slot = tile == t_first ? 0 : 1;
    float tot[MB];
    if constexpr (RMS) {
      // a row's 32 chunk threads are 32 adjacent lanes: xor butterfly
      // (every lane ends with the same bits)
#pragma unroll
      for (int r = 0; r < SPT; ++r) {
        float v = ssr[r];
#pragma unroll
        for (int o = CPR / 2; o > 0; o >>= 1) v += __shfl_xor(v, o);
        if (qc == 0) ssc[tid / CPR + (THREADS / CPR) * r] = v;
        ssr[r] = 0.0f;
      }
      lds_barrier();
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) tot[mb] = ssc[16 * mb + j];
    }
    const int cbase = 16 * wave + 4 * s;  // column of element 0 within the tile
    float* rec_tile = rec + (w_id * 2 + slot) * static_cast<long long>(M) * kCols;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      const int m = 16 * mb + j;
      if (m >= M) continue;
      if (whole) {
        const float scale = RMS ? 1.0f / sqrtf(tot[mb] / static_cast<float>(K) + eps) : 1.0f;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const long long n = tile * kCols + cbase + e;
          if (n < N) y[static_cast<long long>(m) * N + n] = acc[mb][e] * scale;
        }
      } else {
        *reinterpret_cast<floatx4*>(rec_tile + static_cast<long long>(m) * kCols + cbase) = acc[mb];
        if (RMS && wave == 0 && s == 0) rec_ss[(w_id * 2 + slot) * M + m] = tot[mb];
      }
    }
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) acc[mb] = zero4();
  };

  // Prologue: X of unit u0 (loaded before the weights, so the wait for it
  // leaves them in flight), the weights of unit u0, X' of u0 to LDS.
  Cursor cc{u0, t_first, u0 - t_first * upt, row_of(t_first)};  // unit being computed
  Cursor cl = cc;                                                 // next weight load
  XStage S;
  long long xu = u0, xku = u0 - t_first * upt;  // next X to load: unit, unit in its tile
  auto x_next = [&]() __attribute__((always_inline)) {
    load_x(S, xu, xku);
    ++xu;
    if (++xku == upt) xku = 0;
  };
  x_next();
  if constexpr (STAGED) {
    // Unit per iteration from stage b: X and weights of the next unit loaded
    // first, the unit computed, then the next unit's X' and weights written
    // (X' and the weights into the other buffer and stage) and one barrier
    // (two with one X buffer: the rewrite waits until every wave has read
    // it). Every iteration issues the same loads -- past the range the
    // current unit again.
    halfx8 wr[4];
    load_wk(wr, cl);
    advance(cl);
    store_x(S, xbuf[0]);
    put_wk(wr, 0);
    lds_barrier();
    for (int b = 0;; b ^= 1) {
      x_next();
      __builtin_amdgcn_sched_barrier(0);
      load_wk(wr, cl.u < u1 ? cl : cc);
      __builtin_amdgcn_sched_barrier(0);
      compute_kn(xbuf[XB == 2 ? b : 0], b, cc);
      advance(cl);
      if (cc.ku == upt - 1 || cc.u == u1 - 1) finish(cc);
      if (cc.u + 1 < u1) {
        if constexpr (XB == 1) lds_barrier();
        store_x(S, xbuf[XB == 2 ? (b ^ 1) : 0]);
        put_wk(wr, b ^ 1);
      }
      lds_barrier();
      advance(cc);
      if (cc.u >= u1) break;
    }
  } else {
    WV w[LPU];
    load_w(w, cl);
    advance(cl);
    store_x(S, xbuf[0]);
    lds_barrier();

    // One unit per iteration with X' in buffer b: loads X of the next unit
    // first, then computes (reloading w for the next unit load by load),
    // writes the next unit's X' to the other buffer. A single loop body (no
    // unrolling) keeps the weight registers in place across iterations: two
    // copies of the body assigned them differently, and the copies between
    // them waited for every load in flight.
    for (int b = 0;; b ^= 1) {
      x_next();
      __builtin_amdgcn_sched_barrier(0);
      compute(w, xbuf[b], cc, cl);
      advance(cl);
      if (cc.ku == upt - 1 || cc.u == u1 - 1) finish(cc);
      if (cc.u + 1 < u1) store_x(S, xbuf[b ^ 1]);
      lds_barrier();
      advance(cc);
      if (cc.u >= u1) break;
    }
  }
}

// Tiles split between workgroups: y[m][n] = s_m * sum over the tile's
// workgroups, in workgroup order, of their records (s_m = 1 without RMS;
// with RMS from the records' sums of squares, added in the same order).
// One block per (tile, 16 rows): the plan arithmetic runs once per block
// (the same for every thread), thread (r, c4) adds 4 consecutive columns of
// row 16 blockIdx.y + r with one 16-byte load per record, up to 4 records
// in flight. Tiles one workgroup covered whole are skipped (written
// directly).
template <bool RMS>
__global__ __launch_bounds__(256) void skinny_reduce_kernel(const float* __restrict__ rec,
                                                            const float* __restrict__ rec_ss,
                                                            float* __restrict__ y, int M,
                                                            long long N, long long K, Plan plan,
                                                            float eps) {
  const long long tile = blockIdx.x;
  const long long wf = worker_of(tile * plan.upt, plan.U, plan.P);
  const long long wl = worker_of(tile * plan.upt + plan.upt - 1, plan.U, plan.P);
  if (wf == wl) return;  // one workgroup covered the tile: written directly
  const int r = threadIdx.x / 16;
  const int c = 4 * (threadIdx.x % 16);
  const int m = 16 * static_cast<int>(blockIdx.y) + r;
  if (m >= M) return;
  // Every workgroup after wf starts inside the tile (its first tile, slot
  // 0); wf's record is slot 0 only when it starts exactly at the tile.
  const int slot_f = unit_begin(wf, plan.U, plan.P) == tile * plan.upt ? 0 : 1;
  floatx4 v = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
  float tot = 0.0f;
  for (long long w0 = wf; w0 <= wl; w0 += 4) {
    floatx4 p[4];
    float q[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const long long w = w0 + i <= wl ? w0 + i : wl;
      const long long rr = w * 2 + (w == wf ? slot_f : 0);
      p[i] = *reinterpret_cast<const floatx4*>(rec + (rr * M + m) * kCols + c);
      if constexpr (RMS) q[i] = rec_ss[rr * M + m];
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v += w0 + i <= wl ? p[i] : floatx4{0.0f, 0.0f, 0.0f, 0.0f};
      if constexpr (RMS) tot += w0 + i <= wl ? q[i] : 0.0f;
    }
  }
  if constexpr (RMS) v *= 1.0f / sqrtf(tot / static_cast<float>(K) + eps);
  float* yr = y + static_cast<long long>(m) * N + tile * kCols + c;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    if (tile * kCols + c + e < N) yr[e] = v[e];
  }
}

std::size_t scratch_for(const Plan& p, long long M) {
  return static_cast<std::size_t>(p.P) * 2 * M * (kCols + 1) * sizeof(float);
}

// Output-major fp16 W through LDS stages (WMODE 2) at one m-block, straight
// into registers (0) otherwise and for fp32 W: at 11008 x 4096, 16 rows 24.2
// against 27.3 us, 32 rows 33.2 against 33.0, 48 rows 43.3 against 41.2, 64
// rows 52.2 against 49.0 (past 32 rows the staged form keeps one X' buffer
// and two barriers per unit). Both give the same bits.
template <typename WT, int MB>
constexpr int kNkMode = (std::is_same<WT, _Float16>::value && MB == 1) ? 2 : 0;

template <typename WT, bool NK, int MB, bool RMS>
void run_skinny(const SkinnyArgs& a, hipStream_t stream) {
  const long long N = a.N;
  const long long K = a.K;
  const int M = static_cast<int>(a.M);
  const Plan plan = make_plan(N, K, device_cu_count());
  ENG_CHECK(plan.P <= 0x7fffffffLL && plan.tiles <= 0x7fffffffLL,
            "linear: grid too large for one launch");
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
  const unsigned grid = static_cast<unsigned>(plan.P);
  const WT* W = static_cast<const WT*>(a.W);
  if constexpr (NK) {
    skinny_nk_kernel<WT, MB, RMS, kNkMode<WT, MB>><<<grid, kWaves * 64, 0, stream>>>(
        W, a.x, RMS ? a.gamma : nullptr, a.y, M, N, K, plan, rec, rec_ss, a.eps);
  } else if constexpr (std::is_same<WT, _Float16>::value) {
    skinny_nk_kernel<WT, MB, RMS, 1><<<grid, kWaves * 64, 0, stream>>>(
        W, a.x, RMS ? a.gamma : nullptr, a.y, M, N, K, plan, rec, rec_ss, a.eps);
  } else {
    skinny_mfma_kernel<WT, NK, MB, RMS><<<grid, kWaves * 64, 0, stream>>>(
        W, a.x, a.gamma, a.y, M, N, K, plan, rec, rec_ss, a.eps);
  }
  ENG_LAUNCH_CHECK();
  // Every workgroup takes whole tiles: nothing left to add.
  if (plan.U % plan.P == 0 && (plan.U / plan.P) % plan.upt == 0) return;
  skinny_reduce_kernel<RMS><<<dim3(static_cast<unsigned>(plan.tiles), (M + 15) / 16), 256, 0, stream>>>(
      rec, rec_ss, a.y, M, N, K, plan, a.eps);
  ENG_LAUNCH_CHECK();
}

template <typename WT, bool NK, bool RMS>
void dispatch_mb(const SkinnyArgs& a, hipStream_t stream) {
  if constexpr (std::is_same<WT, _Float16>::value) {  // at most 32 rows
    if (a.M <= 16)
      run_skinny<WT, NK, 1, RMS>(a, stream);
    else
      run_skinny<WT, NK, 2, RMS>(a, stream);
  } else {
    switch ((a.M + 15) / 16) {
      case 1: run_skinny<WT, NK, 1, RMS>(a, stream); break;
      case 2: run_skinny<WT, NK, 2, RMS>(a, stream); break;
      case 3: run_skinny<WT, NK, 3, RMS>(a, stream); break;
      default: run_skinny<WT, NK, 4, RMS>(a, stream); break;
    }
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
  if (a.M < kSkinnyMinRows || a.M > (a.w == Elem::F16 ? kSkinnyMaxRowsF16 : kSkinnyMaxRows))
    return false;
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
