// gemm.hip -- FP32 GEMM on gfx950 matrix cores (C[M x N] = A[M x K] . B[K x N]).
//
// Replaces the SIMT register-tiled kernel behind matmul_register_tiled
// (reference kernels/matmul_register_tiled.cu:48-199) and serves the M > 1
// case of rmsnorm_linear (reference kernels/rmsnorm_linear.cu:195-199), with
// the RMSNorm fused in: gamma scales A's columns as they are staged, the row
// sums of squares are accumulated from the same staged values, and the row
// scale multiplies the accumulators in the epilogue.
//
// Tiling for wave64 and v_mfma_f32_32x32x2_f32:
//   * workgroup tile 128 x 128, K step 32, 256 threads = 4 waves in 2 x 2;
//   * each wave owns 64 x 64 = 2 x 2 MFMA blocks of 32 x 32 (64 fp32
//     accumulators per lane);
//   * operand layout of the instruction: lane l supplies A[l % 32][k] and
//     B[k][l % 32] with k = l / 32 of the pair; accumulator v of lane l is
//     C[8 (v / 4) + 4 (l / 32) + v % 4][l % 32]. Within a 32-deep K tile the
//     instruction at step s pairs k = s (lanes 0-31) with k = 16 + s (lanes
//     32-63), so each lane reads a contiguous 16-float run of its A row
//     (ds_read_b128) and a 16-row column of B (ds_read_b32, conflict-free);
//   * A and B tiles are double-buffered in LDS with 4-float row padding; the
//     next tile's global loads are issued before the current tile's MFMAs;
//   * the workgroup -> tile map is XCD-aware: consecutive workgroup ids go to
//     different XCDs, so ids are regrouped so each XCD works on a contiguous
//     band of tiles (grouped 8 tile-rows deep) and shares A/B panels in its L2.
#include "launch.hpp"

#include <algorithm>
#include <type_traits>

namespace eng {
namespace {

typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef _Float16 halfx8 __attribute__((ext_vector_type(8)));

constexpr int BM = 128;
constexpr int BN = 128;
constexpr int BK = 32;
constexpr int kThreads = 256;
constexpr int AS = BK + 4;   // A tile row stride in LDS (floats)
constexpr int BS = BN + 4;   // B tile row stride in LDS (floats)
constexpr int kGroupM = 8;   // tile-rows per raster group
constexpr int kXcds = 8;

// Global -> register staging of a B tile, K x N layout (B[k][n], rows along N):
// 32 rows of 128 elements.
template <typename BT>
struct BLoad;
template <>
struct BLoad<float> {
  static constexpr int kLoads = 4;   // 4 x float4 per thread
  static constexpr int kVec = 4;
  static constexpr int kThreadsPerRow = BN / kVec;                // 32
  static constexpr int kRowsPerLoad = kThreads / kThreadsPerRow;  // 8
};
template <>
struct BLoad<_Float16> {
  static constexpr int kLoads = 2;   // 2 x 8 halves per thread
  static constexpr int kVec = 8;
  static constexpr int kThreadsPerRow = BN / kVec;                // 16
  static constexpr int kRowsPerLoad = kThreads / kThreadsPerRow;  // 16
};

// Staging of a B tile given N x K (B^T[n][k], rows along K): 128 rows of 32
// elements, the same shape as an A tile.
template <typename BT>
struct BtLoad;
template <>
struct BtLoad<float> {
  static constexpr int kLoads = 4;
  static constexpr int kVec = 4;
  static constexpr int kThreadsPerRow = BK / kVec;                // 8
  static constexpr int kRowsPerLoad = kThreads / kThreadsPerRow;  // 32
};
template <>
struct BtLoad<_Float16> {
  static constexpr int kLoads = 2;
  static constexpr int kVec = 8;
  static constexpr int kThreadsPerRow = BK / kVec;                // 4
  static constexpr int kRowsPerLoad = kThreads / kThreadsPerRow;  // 64
};

// Workgroup id -> (tile_m, tile_n). Workgroups are handed to XCDs round-robin,
// so id w runs on XCD w % 8; renumber so XCD x gets a contiguous logical range,
// then raster that range in groups of kGroupM tile-rows.
__device__ __forceinline__ void tile_of(int wg, int tiles_m, int tiles_n, int& tm, int& tn) {
  const int ntiles = tiles_m * tiles_n;
  const int q = ntiles / kXcds;
  const int r = ntiles % kXcds;
  const int xcd = wg % kXcds;
  const int local = wg / kXcds;
  const int logical = xcd * q + (xcd < r ? xcd : r) + local;
  const int group_size = kGroupM * tiles_n;
  const int group = logical / group_size;
  const int first_m = group * kGroupM;
  const int gm = (tiles_m - first_m) < kGroupM ? (tiles_m - first_m) : kGroupM;
  const int in_group = logical - group * group_size;
  tm = first_m + in_group % gm;
  tn = in_group / gm;
}

// BNK: B is given as B^T, row-major [N x K]; its tile is staged like an A
// tile (n rows, k contiguous) and its fragments are read like A's.
template <typename BT, bool BNK, bool VA, bool VB, bool RMS>
__global__ __launch_bounds__(kThreads, 2) void gemm_f32_mfma_kernel(
    const float* __restrict__ A, const BT* __restrict__ B, float* __restrict__ C,
    const float* __restrict__ gamma, int M, int N, int K, float eps, int tiles_m, int tiles_n) {
  using BL = typename std::conditional<BNK, BtLoad<BT>, BLoad<BT>>::type;
  constexpr int kBTile = BNK ? BN * AS : BK * BS;
  __shared__ __attribute__((aligned(16))) float As[2][BM * AS];
  __shared__ __attribute__((aligned(16))) float Bs[2][kBTile];
  __shared__ float row_scale[RMS ? BM : 1];

  const int t = threadIdx.x;
  const int lane = t & 63;
  const int wave = t >> 6;
  const int li = lane & 31;  // row (A) / column (B, C) inside a 32 x 32 block
  const int lg = lane >> 5;  // which half of the K pair
  const int wm = wave >> 1;
  const int wn = wave & 1;

  int tm, tn;
  tile_of(blockIdx.x, tiles_m, tiles_n, tm, tn);
  const int m0 = tm * BM;
  const int n0 = tn * BN;

  // Global -> register staging assignments.
  const int a_row = t >> 3;        // + 32 * i
  const int a_col = (t & 7) * 4;   // k offset inside the tile
  const int b_row = t / BL::kThreadsPerRow;            // + kRowsPerLoad * i
  const int b_col = (t % BL::kThreadsPerRow) * BL::kVec;

  floatx4 ra[4];
  float rb[BL::kLoads][BL::kVec];
  float ss[4] = {0.0f, 0.0f, 0.0f, 0.0f};

  auto load_a = [&](int k0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = m0 + a_row + 32 * i;
      const int kc = k0 + a_col;
      floatx4 v = {0.0f, 0.0f, 0.0f, 0.0f};
      if (row < M) {
        const float* src = A + static_cast<long long>(row) * K + kc;
        if constexpr (VA) {
          if (kc < K) v = *reinterpret_cast<const floatx4*>(src);
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (kc + e < K) v[e] = src[e];
        }
      }
      ra[i] = v;
    }
  };

  auto load_b = [&](int k0) {
#pragma unroll
    for (int i = 0; i < BL::kLoads; ++i) {
#pragma unroll
      for (int e = 0; e < BL::kVec; ++e) rb[i][e] = 0.0f;
      if constexpr (BNK) {
        const int n = n0 + b_row + BL::kRowsPerLoad * i;
        const int kc = k0 + b_col;
        if (n < N) {
          const BT* src = B + static_cast<long long>(n) * K + kc;
          if constexpr (VB) {
            if (kc < K) {
              if constexpr (BL::kVec == 4) {
                const floatx4 v = *reinterpret_cast<const floatx4*>(src);
#pragma unroll
                for (int e = 0; e < 4; ++e) rb[i][e] = v[e];
              } else {
                const halfx8 v = *reinterpret_cast<const halfx8*>(src);
#pragma unroll
                for (int e = 0; e < 8; ++e) rb[i][e] = static_cast<float>(v[e]);
              }
            }
          } else {
#pragma unroll
            for (int e = 0; e < BL::kVec; ++e)
              if (kc + e < K) rb[i][e] = static_cast<float>(src[e]);
          }
        }
        continue;
      }
      const int krow = k0 + b_row + BL::kRowsPerLoad * i;
      const int nc = n0 + b_col;
      if (krow < K) {
        const BT* src = B + static_cast<long long>(krow) * N + nc;
        if constexpr (VB) {
          if (nc < N) {
            if constexpr (BL::kVec == 4) {
              const floatx4 v = *reinterpret_cast<const floatx4*>(src);
#pragma unroll
              for (int e = 0; e < 4; ++e) rb[i][e] = v[e];
            } else {
              const halfx8 v = *reinterpret_cast<const halfx8*>(src);
#pragma unroll
              for (int e = 0; e < 8; ++e) rb[i][e] = static_cast<float>(v[e]);
            }
          }
        } else {
#pragma unroll
          for (int e = 0; e < BL::kVec; ++e)
            if (nc + e < N) rb[i][e] = static_cast<float>(src[e]);
        }
      }
    }
  };

  auto store_tiles = [&](int buf, int k0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      floatx4 v = ra[i];
      if constexpr (RMS) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          ss[i] = fmaf(v[e], v[e], ss[i]);
          const int k = k0 + a_col + e;
          if (gamma != nullptr && k < K) v[e] *= gamma[k];
        }
      }
      *reinterpret_cast<floatx4*>(&As[buf][(a_row + 32 * i) * AS + a_col]) = v;
    }
#pragma unroll
    for (int i = 0; i < BL::kLoads; ++i) {
      float* dst = &Bs[buf][(b_row + BL::kRowsPerLoad * i) * (BNK ? AS : BS) + b_col];
#pragma unroll
      for (int e = 0; e < BL::kVec; e += 4) {
        const floatx4 v = {rb[i][e], rb[i][e + 1], rb[i][e + 2], rb[i][e + 3]};
        *reinterpret_cast<floatx4*>(dst + e) = v;
      }
    }
  };

  floatx16 acc[2][2];
#pragma unroll
  for (int mb = 0; mb < 2; ++mb)
#pragma unroll
    for (int nb = 0; nb < 2; ++nb)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[mb][nb][v] = 0.0f;

  const int nk = (K + BK - 1) / BK;
  load_a(0);
  load_b(0);
  store_tiles(0, 0);
  __syncthreads();

  for (int kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < nk) {
      load_a((kt + 1) * BK);
      load_b((kt + 1) * BK);
    }

    // This wave's operand fragments for the whole 32-deep tile.
    floatx4 af[2][4];
#pragma unroll
    for (int mb = 0; mb < 2; ++mb) {
      const float* src = &As[cur][(wm * 64 + mb * 32 + li) * AS + lg * 16];
#pragma unroll
      for (int q = 0; q < 4; ++q) af[mb][q] = *reinterpret_cast<const floatx4*>(src + 4 * q);
    }
    float bf[2][16];
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
      if constexpr (BNK) {
        const float* src = &Bs[cur][(wn * 64 + nb * 32 + li) * AS + lg * 16];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const floatx4 v = *reinterpret_cast<const floatx4*>(src + 4 * q);
#pragma unroll
          for (int e = 0; e < 4; ++e) bf[nb][4 * q + e] = v[e];
        }
      } else {
        const float* src = &Bs[cur][(lg * 16) * BS + wn * 64 + nb * 32 + li];
#pragma unroll
        for (int s = 0; s < 16; ++s) bf[nb][s] = src[s * BS];
      }
    }
#pragma unroll
    for (int s = 0; s < 16; ++s) {
#pragma unroll
      for (int mb = 0; mb < 2; ++mb) {
        const float a = af[mb][s >> 2][s & 3];
#pragma unroll
        for (int nb = 0; nb < 2; ++nb)
          acc[mb][nb] = __builtin_amdgcn_mfma_f32_32x32x2f32(a, bf[nb][s], acc[mb][nb], 0, 0, 0);
      }
    }

    if (kt + 1 < nk) store_tiles(cur ^ 1, (kt + 1) * BK);
    __syncthreads();
  }

  if constexpr (RMS) {
    // The 8 lanes t..t+7 staged the same A row: fold their sums of squares.
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float v = ss[i];
      v += __shfl_xor(v, 1);
      v += __shfl_xor(v, 2);
      v += __shfl_xor(v, 4);
      if ((t & 7) == 0) row_scale[a_row + 32 * i] = 1.0f / sqrtf(v / static_cast<float>(K) + eps);
    }
    __syncthreads();
  }

#pragma unroll
  for (int mb = 0; mb < 2; ++mb) {
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
      const int col = n0 + wn * 64 + nb * 32 + li;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int rl = wm * 64 + mb * 32 + 8 * (v >> 2) + 4 * lg + (v & 3);
        const int row = m0 + rl;
        if (row < M && col < N) {
          float out = acc[mb][nb][v];
          if constexpr (RMS) out *= row_scale[rl];
          C[static_cast<long long>(row) * N + col] = out;
        }
      }
    }
  }
}

template <typename BT, bool BNK, bool RMS>
void run_gemm(const GemmArgs& a, hipStream_t stream) {
  constexpr int kBVec = 16 / static_cast<int>(sizeof(BT));
  const bool va = (a.K % 4 == 0) && aligned_to(a.A, 16);
  // B rows run along N ([K x N]) or along K ([N x K]).
  const bool vb = ((BNK ? a.K : a.N) % kBVec == 0) && aligned_to(a.B, 16);
  const int M = static_cast<int>(a.M);
  const int N = static_cast<int>(a.N);
  const int K = static_cast<int>(a.K);
  const int tiles_m = (M + BM - 1) / BM;
  const int tiles_n = (N + BN - 1) / BN;
  const long long ntiles = static_cast<long long>(tiles_m) * tiles_n;
  ENG_CHECK(ntiles <= 0x7fffffffLL, "matmul: too many tiles for one launch");
  const dim3 grid(static_cast<unsigned>(ntiles));
  const BT* B = static_cast<const BT*>(a.B);
#define ENG_GEMM_LAUNCH(VA_, VB_)                                                       \
  gemm_f32_mfma_kernel<BT, BNK, VA_, VB_, RMS><<<grid, kThreads, 0, stream>>>(          \
      a.A, B, a.C, a.gamma, M, N, K, a.eps, tiles_m, tiles_n)
  if (va && vb) {
    ENG_GEMM_LAUNCH(true, true);
  } else if (va) {
    ENG_GEMM_LAUNCH(true, false);
  } else if (vb) {
    ENG_GEMM_LAUNCH(false, true);
  } else {
    ENG_GEMM_LAUNCH(false, false);
  }
#undef ENG_GEMM_LAUNCH
  ENG_LAUNCH_CHECK();
}

template <typename BT, bool BNK>
void run_gemm_rms(const GemmArgs& a, hipStream_t stream) {
  if (a.rms) {
    run_gemm<BT, BNK, true>(a, stream);
  } else {
    run_gemm<BT, BNK, false>(a, stream);
  }
}

}  // namespace

void launch_gemm(const GemmArgs& a, hipStream_t stream) {
  ENG_CHECK(a.M <= 0x7fffffffLL && a.N <= 0x7fffffffLL && a.K <= 0x7fffffffLL,
            "matmul: dimensions must fit in 31 bits");
  if (a.b == Elem::F32) {
    if (a.b_nk) {
      run_gemm_rms<float, true>(a, stream);
    } else {
      run_gemm_rms<float, false>(a, stream);
    }
  } else {
    if (a.b_nk) {
      run_gemm_rms<_Float16, true>(a, stream);
    } else {
      run_gemm_rms<_Float16, false>(a, stream);
    }
  }
}

}  // namespace eng

using eng::guarded;

extern "C" {

int eng_matmul_f32(const float* A, const float* B, float* C, int64_t M, int64_t N, int64_t K,
                   eng_stream stream) {
  return guarded([&] {
    ENG_CHECK(A != nullptr, "matmul_register_tiled: A is null");
    ENG_CHECK(B != nullptr, "matmul_register_tiled: B is null");
    ENG_CHECK(C != nullptr, "matmul_register_tiled: C is null");
    ENG_CHECK(M >= 0, "matmul_register_tiled: M must be non-negative");
    ENG_CHECK(N >= 0, "matmul_register_tiled: N must be non-negative");
    ENG_CHECK(K >= 0, "matmul_register_tiled: K must be non-negative");
    if (M == 0 || N == 0) return;
    hipStream_t s = eng::as_stream(stream);
    // An M x 0 times 0 x N product is the M x N zero matrix.
    if (K == 0) {
      eng::fill_zero_async(C, static_cast<std::size_t>(M) * static_cast<std::size_t>(N) *
                                  sizeof(float),
                           s);
      return;
    }
    if (M == 1) {
      // A single row is a GEMV: out[N] = A[0][K] . B[K x N].
      eng::GemvArgs g;
      g.W = B;
      g.w = eng::Elem::F32;
      g.x = A;
      g.y = C;
      g.N = N;
      g.K = K;
      eng::launch_gemv(g, s);
      return;
    }
    eng::GemmArgs g;
    g.A = A;
    g.B = B;
    g.C = C;
    g.M = M;
    g.N = N;
    g.K = K;
    eng::launch_gemm(g, s);
  });
}

}  // extern "C"
