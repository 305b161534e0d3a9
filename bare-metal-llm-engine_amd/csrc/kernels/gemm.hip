// gemm.hip -- FP32 GEMM on gfx950 matrix cores (C[M x N] = A[M x K] . B[K x N]).
//
// Replaces the SIMT register-tiled kernel behind matmul_register_tiled
// (reference kernels/matmul_register_tiled.cu:48-199); it is also the M > 1
// half of rmsnorm_linear, which, as in the reference
// (kernels/rmsnorm_linear.cu:191-199), normalises the rows into scratch
// first. (Fusing the RMSNorm into this kernel -- gamma applied to the A
// fragments, row sums of squares taken from them -- measured 30% slower than
// the separate pass at 512 x 4096 x 4096: every N-tile repeats the multiply,
// and it sits between the LDS read and the MFMA.)
//
// Tiling for wave64 and v_mfma_f32_32x32x2_f32:
//   * workgroup tile BM x BN (256 x 128, 128 x 128, 128 x 64 or 64 x 64), K
//     step 32; 256 x 128 runs 512 threads = 8 waves in 4 x 2 with three LDS
//     stages, one workgroup per CU, the others 256 threads = 4 waves in 2 x 2
//     with two stages, two workgroups per CU; each wave owns its block of the
//     tile as 32 x 32 MFMA blocks;
//   * operand layout of the instruction: lane l supplies A[l % 32][k] and
//     B[k][l % 32] with k = l / 32 of the pair; accumulator v of lane l is
//     C[8 (v / 4) + 4 (l / 32) + v % 4][l % 32]. Within a 32-deep K tile the
//     instruction at step s pairs k = s (lanes 0-31) with k = 16 + s (lanes
//     32-63), so each lane reads a contiguous 16-float run of its A row
//     (ds_read_b128) and a 16-row column of B (ds_read_b32, conflict-free) --
//     or, when B is given transposed ([N x K]), a 16-float run of its B row;
//   * operands with K % 32 == 0 and 16-byte aligned rows take
//     gemm_f32_mfma_dma_kernel, which loads tiles straight into LDS (below;
//     fp16 B is converted as fragments are read; ragged M / N clamp their edge
//     loads); the rest take gemm_f32_mfma_kernel, which stages through registers: A and B tiles are
//     double-buffered in LDS with 4-float row padding and the next tile's
//     global loads are issued before the current tile's MFMAs;
//   * the workgroup -> tile map is XCD-aware: consecutive workgroup ids go to
//     different XCDs, so ids are regrouped so each XCD works on a contiguous
//     band of tiles (grouped 8 tile-rows deep) and shares A/B panels in its L2;
//   * the tile shape is chosen per call so the grid covers the 256 CUs evenly
//     (small-M shapes such as 512 x 4096 x 11008 would leave half the CUs idle
//     with 128 x 128 tiles);
//   * fragments are read a quarter K tile (4 MFMA k-slices) ahead of the
//     MFMAs that use them.
#include "launch.hpp"

#include <algorithm>
#include <cstdlib>
#include <type_traits>

namespace eng {
namespace {

typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef _Float16 halfx8 __attribute__((ext_vector_type(8)));

constexpr int BK = 32;
constexpr int kThreads = 256;
constexpr int AS = BK + 4;   // row stride (floats) of k-contiguous tiles in LDS
constexpr int kGroupM = 8;   // tile-rows per raster group
constexpr int kXcds = 8;

// Global -> register staging of a B tile: 16-byte vectors, `kLoads` per thread.
// K x N layout: BK rows of BN elements; N x K layout: BN rows of BK elements.
template <typename BT, bool BNK, int BN>
struct BStage {
  static constexpr int kVec = 16 / static_cast<int>(sizeof(BT));
  static constexpr int kRowLen = BNK ? BK : BN;
  static constexpr int kThreadsPerRow = kRowLen / kVec;
  static constexpr int kRowsPerLoad = kThreads / kThreadsPerRow;
  static constexpr int kLoads = (BNK ? BN : BK) / kRowsPerLoad;
  static_assert(kLoads >= 1 && kLoads * kRowsPerLoad == (BNK ? BN : BK), "B staging shape");
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
template <int BM, int BN, typename BT, bool BNK, bool VA, bool VB>
__global__ __launch_bounds__(kThreads, 2) void gemm_f32_mfma_kernel(
    const float* __restrict__ A, const BT* __restrict__ B, float* __restrict__ C, int M, int N,
    int K, int tiles_m, int tiles_n) {
  using BL = BStage<BT, BNK, BN>;
  constexpr int WM = BM / 2;       // rows per wave
  constexpr int WN = BN / 2;       // columns per wave
  constexpr int MB = WM / 32;      // MFMA blocks per wave, along M
  constexpr int NB = WN / 32;      // ... along N
  constexpr int A_LOADS = BM / 32; // float4 A loads per thread per K tile
  constexpr int BSK = BN + 4;      // row stride of a K x N B tile
  constexpr int kBTile = BNK ? BN * AS : BK * BSK;
  __shared__ __attribute__((aligned(16))) float As[2][BM * AS];
  __shared__ __attribute__((aligned(16))) float Bs[2][kBTile];

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

  floatx4 ra[A_LOADS];
  float rb[BL::kLoads][BL::kVec];

  auto load_a = [&](int k0) {
#pragma unroll
    for (int i = 0; i < A_LOADS; ++i) {
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
      // (r, c): row and first column of this thread's vector in B's storage.
      const int r = (BNK ? n0 : k0) + b_row + BL::kRowsPerLoad * i;
      const int c = (BNK ? k0 : n0) + b_col;
      const int rows = BNK ? N : K;
      const int cols = BNK ? K : N;
      if (r < rows) {
        const BT* src = B + static_cast<long long>(r) * cols + c;
        if constexpr (VB) {
          if (c < cols) {
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
            if (c + e < cols) rb[i][e] = static_cast<float>(src[e]);
        }
      }
    }
  };

  auto store_tiles = [&](int buf) {
#pragma unroll
    for (int i = 0; i < A_LOADS; ++i)
      *reinterpret_cast<floatx4*>(&As[buf][(a_row + 32 * i) * AS + a_col]) = ra[i];
#pragma unroll
    for (int i = 0; i < BL::kLoads; ++i) {
      float* dst = &Bs[buf][(b_row + BL::kRowsPerLoad * i) * (BNK ? AS : BSK) + b_col];
#pragma unroll
      for (int e = 0; e < BL::kVec; e += 4) {
        const floatx4 v = {rb[i][e], rb[i][e + 1], rb[i][e + 2], rb[i][e + 3]};
        *reinterpret_cast<floatx4*>(dst + e) = v;
      }
    }
  };

  floatx16 acc[MB][NB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[mb][nb][v] = 0.0f;

  const int nk = (K + BK - 1) / BK;
  load_a(0);
  load_b(0);
  store_tiles(0);
  __syncthreads();

  for (int kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < nk) {
      load_a((kt + 1) * BK);
      load_b((kt + 1) * BK);
    }

    // This wave's operand fragments for the whole 32-deep tile.
    floatx4 af[MB][4];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      const float* src = &As[cur][(wm * WM + mb * 32 + li) * AS + lg * 16];
#pragma unroll
      for (int q = 0; q < 4; ++q) af[mb][q] = *reinterpret_cast<const floatx4*>(src + 4 * q);
    }
    float bf[NB][16];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      if constexpr (BNK) {
        const float* src = &Bs[cur][(wn * WN + nb * 32 + li) * AS + lg * 16];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const floatx4 v = *reinterpret_cast<const floatx4*>(src + 4 * q);
#pragma unroll
          for (int e = 0; e < 4; ++e) bf[nb][4 * q + e] = v[e];
        }
      } else {
        const float* src = &Bs[cur][(lg * 16) * BSK + wn * WN + nb * 32 + li];
#pragma unroll
        for (int s = 0; s < 16; ++s) bf[nb][s] = src[s * BSK];
      }
    }
#pragma unroll
    for (int s = 0; s < 16; ++s) {
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        const float a = af[mb][s >> 2][s & 3];
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
          acc[mb][nb] = __builtin_amdgcn_mfma_f32_32x32x2f32(a, bf[nb][s], acc[mb][nb], 0, 0, 0);
      }
    }

    if (kt + 1 < nk) store_tiles(cur ^ 1);
    __syncthreads();
  }

#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      const int col = n0 + wn * WN + nb * 32 + li;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int row = m0 + wm * WM + mb * 32 + 8 * (v >> 2) + 4 * lg + (v & 3);
        if (row < M && col < N) C[static_cast<long long>(row) * N + col] = acc[mb][nb][v];
      }
    }
  }
}

// Variant fed by direct global -> LDS loads (buffer_load_dwordx4 ... lds:
// lane l of a wave writes 16 bytes at the wave's LDS base + 16 l, from the
// offset the lane names past the descriptor's base). No staging registers and
// no LDS store instructions: a stage's loads are issued one or two K tiles
// before it is read and land while the MFMAs run; one s_waitcnt and one
// barrier hand each stage over. LDS tiles are unpadded and the 16-byte chunk
// positions are XOR-swizzled instead, which the fetch side applies by choosing
// which global chunk each lane loads:
//   * k-contiguous tiles (A, and B given [N x K]): chunk c of row r sits at
//     c ^ ((r >> 1) & 7), so the 16 rows a 16-lane slice of ds_read_b128
//     touches fall in 16 distinct bank groups;
//   * [K x N] B tiles: chunk c of row k sits at c ^ (8 ((k >> 4) & 1)), so the
//     rows k and k + 16 read by the two half-waves of a ds_read_b32 use
//     disjoint banks.
// Requires K % 32 == 0 and 16-byte aligned A and B (ragged M / N: EDGE below).
__device__ __forceinline__ int swz_rows(int r) { return (r >> 1) & 7; }

// 16-byte direct load into LDS through a buffer descriptor: lane l reads the
// bytes [off, off + 16) past base and writes them to lds + 16 l (lds the same
// in every lane of the wave). The descriptor covers `bytes` bytes from base
// (reads past them return zeros). base must be wave-uniform. Buffer loads,
// unlike global_load_lds, are not FLAT instructions: the compiler then counts
// the in-flight direct loads on vmcnt only and keeps the LDS fragment reads'
// waits partial instead of draining them with lgkmcnt(0).
[[maybe_unused]] constexpr int kRsrcWord3 = 0x00020000;  // gfx9 buffer descriptor word 3 (raw dword access)

template <typename T>
__device__ __forceinline__ void lds_buf16(const T* base, unsigned bytes, unsigned off, T* lds) {
#if defined(__HIP_DEVICE_COMPILE__)
  __builtin_amdgcn_raw_ptr_buffer_load_lds(
      __builtin_amdgcn_make_buffer_rsrc(const_cast<T*>(base), 0, static_cast<int>(bytes), kRsrcWord3),
      lds, 16, static_cast<int>(off), 0, 0, 0);
#endif
}

// Bytes from element `from` to the end of an n-element array, capped at the
// 32-bit range of a buffer descriptor.
template <typename T>
__device__ __forceinline__ unsigned bytes_left(long long n, long long from) {
  const unsigned long long b = static_cast<unsigned long long>(n - from) * sizeof(T);
  return (b >> 32) != 0 ? 0xFFFFFFFFu : static_cast<unsigned>(b);
}

// Waits until this wave's outstanding memory operations, the direct LDS loads
// included, have completed.
__device__ __forceinline__ void wait_all_memory() {
#if defined(__HIP_DEVICE_COMPILE__)
  __builtin_amdgcn_s_waitcnt(0);
#endif
}

// Stage hand-over inside the K loop: waits until at most `vm` of this wave's
// vector-memory operations (direct LDS loads, issued and completing in order)
// are outstanding and all of its LDS reads have returned, then joins the
// workgroup barrier. The barrier is the bare instruction rather than
// __syncthreads(), whose release fence would drain every outstanding load
// (vmcnt(0)) and so cap the ring at one tile in flight; the empty asm
// statements keep the compiler from moving memory accesses across it.
template <int VM>
__device__ __forceinline__ void stage_barrier() {
  static_assert(VM >= 0 && VM < 64, "vmcnt field");
#if defined(__HIP_DEVICE_COMPILE__)
  // gfx9 s_waitcnt: vmcnt bits 3:0 and 15:14, expcnt 6:4 (7 = no wait),
  // lgkmcnt 11:8 (0 = wait for all)
  __builtin_amdgcn_s_waitcnt((VM & 0xF) | ((VM >> 4) << 14) | (0x7 << 4));
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
#endif
}
__device__ __forceinline__ int swz_kn(int k) { return ((k >> 4) & 1) * 8; }
// fp16 B tiles (8 halves per 16-byte chunk). [N x K]: a 32-deep row is 4
// chunks; chunk c of row r sits at c ^ ((r >> 2) & 3), so the 16 rows of a
// 16-lane slice of ds_read_b128 (row pitch 64 bytes) cover all 64 banks.
// [K x N]: chunk c of row k sits at c ^ (4 ((k >> 4) & 1)), moving rows k and
// k + 16 (the two half-waves of a fragment read) 64 bytes apart in the banks.
__device__ __forceinline__ int swz_rows_h(int r) { return (r >> 2) & 3; }
__device__ __forceinline__ int swz_kn_h(int k) { return ((k >> 4) & 1) * 4; }

//
// Workgroup layout: WGM x WGN waves, each owning a (BM / WGM) x (BN / WGN)
// block of the tile as 32 x 32 MFMA blocks, and S LDS stages per operand.
// 128 x 128 and smaller tiles: 4 waves, 2 stages (64 KB for 128 x 128 fp32),
// two workgroups per CU. 256 x 128: 8 waves, 3 stages (144 KB), one
// workgroup per CU; a stage's loads then have two K tiles of MFMAs to land
// in, and each byte loaded feeds a third more MFMA work than on 128 x 128.
template <int BM, int BN>
struct TileCfg {
  static constexpr bool kBig = BM == 256;
  static constexpr int WGM = kBig ? 4 : 2;
  static constexpr int WGN = 2;
  static constexpr int kWaves = WGM * WGN;
  static constexpr int kThreads = 64 * kWaves;
  static constexpr int S = kBig ? 3 : 2;
  static constexpr int kMinBlocks = kBig ? 1 : 2;  // workgroups per CU
  static constexpr int WM = BM / WGM;
  static constexpr int WN = BN / WGN;
  static constexpr int MB = WM / 32;
  static constexpr int NB = WN / 32;
  static_assert(WM % 32 == 0 && WN % 32 == 0, "wave tile");
};

template <int BM, int BN>
using TileAcc = floatx16[TileCfg<BM, BN>::MB][TileCfg<BM, BN>::NB];

// The stages of each operand are separate LDS variables and the K loop is
// unrolled by S, so every LDS access names its buffer statically: the
// compiler tracks direct loads per variable, and a fragment read of one stage
// then waits only for that stage's loads, not for the ones in flight into the
// others.
//
// B may also be fp16 (BT = _Float16): its tiles are loaded into LDS as raw
// halves, half the bytes of an fp32 tile, and converted to fp32 as each lane
// reads its fragment, so the MFMAs and the accumulation are those of the fp32
// path (fp16 -> fp32 is exact).
//
// EDGE: M and N need not be multiples of the tile. Loads of rows (A, [N x K]
// B) or 16-byte column chunks ([K x N] B) past the matrix read the last valid
// one instead -- in bounds, and only ever multiplied into accumulators whose
// C element is outside the matrix -- and those elements are not stored.
//
// The K tiles [kt0, kt1) of the output tile at (m0, n0), accumulated into
// acc (zeroed here); ends with a barrier, so a following call may refill
// the LDS stages.
template <int BM, int BN, bool BNK, typename BT, bool EDGE>
__device__ __forceinline__ void dma_tile(const float* __restrict__ A, const BT* __restrict__ B,
                                         int M, int N, int K, int m0, int n0, int kt0, int kt1,
                                         TileAcc<BM, BN>& acc) {
  using C = TileCfg<BM, BN>;
  constexpr bool HB = std::is_same<BT, _Float16>::value;
  constexpr int BV = 16 / static_cast<int>(sizeof(BT));  // B elements per 16-byte chunk
  constexpr int S = C::S;
  constexpr int MB = C::MB;
  constexpr int NB = C::NB;
  constexpr int A_CH = BM * BK / 4;  // 16-byte chunks of an A tile
  constexpr int B_CH = BN * BK / BV;
  constexpr int A_INST = A_CH / C::kThreads;  // chunk loads per thread (= per wave instruction count)
  constexpr int B_INST = B_CH / C::kThreads;
  constexpr int kLoads = A_INST + B_INST;     // direct loads per thread per K tile
  constexpr int BROW = BN / BV;               // chunks per [K x N] B row
  static_assert(A_CH % C::kThreads == 0 && B_CH % C::kThreads == 0, "tile shape");
  static_assert(S == 2 || S == 3, "stages");
  __shared__ __attribute__((aligned(1024))) float As0[BM * BK];
  __shared__ __attribute__((aligned(1024))) float As1[BM * BK];
  __shared__ __attribute__((aligned(1024))) float As2[S > 2 ? BM * BK : 1];
  __shared__ __attribute__((aligned(1024))) BT Bs0[BN * BK];
  __shared__ __attribute__((aligned(1024))) BT Bs1[BN * BK];
  __shared__ __attribute__((aligned(1024))) BT Bs2[S > 2 ? BN * BK : 1];
  auto a_stage = [&](auto st) -> float* {
    if constexpr (decltype(st)::value == 0) return As0;
    else if constexpr (decltype(st)::value == 1) return As1;
    else return As2;
  };
  auto b_stage = [&](auto st) -> BT* {
    if constexpr (decltype(st)::value == 0) return Bs0;
    else if constexpr (decltype(st)::value == 1) return Bs1;
    else return Bs2;
  };

  const int t = threadIdx.x;
  const int lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int li = lane & 31;
  const int lg = lane >> 5;
  const int wm = wave / C::WGN;
  const int wn = wave % C::WGN;

  // Direct loads of K tile kt into one stage. Wave w's j-th instruction fills
  // chunk slots (waves j + w) * 64 + lane. Each lane's byte offset from the
  // tile's corner is the same for every K tile (a_off, b_off); only the
  // descriptor's base moves, by BK columns of A and BK rows (or columns) of B.
  unsigned a_off[A_INST];
  unsigned b_off[B_INST];
#pragma unroll
  for (int j = 0; j < A_INST; ++j) {
    const int slot = (C::kWaves * j + wave) * 64 + lane;
    const int r = slot >> 3;
    const int c = (slot & 7) ^ swz_rows(r);
    const int row = EDGE ? min(m0 + r, M - 1) - m0 : r;
    a_off[j] = static_cast<unsigned>(row * K + 4 * c) * 4u;
  }
#pragma unroll
  for (int j = 0; j < B_INST; ++j) {
    const int slot = (C::kWaves * j + wave) * 64 + lane;
    if constexpr (BNK) {
      const int r = HB ? slot >> 2 : slot >> 3;
      const int c = HB ? (slot & 3) ^ swz_rows_h(r) : (slot & 7) ^ swz_rows(r);
      const int row = EDGE ? min(n0 + r, N - 1) - n0 : r;
      b_off[j] = static_cast<unsigned>(row * K + BV * c) * static_cast<unsigned>(sizeof(BT));
    } else {
      const int k = slot / BROW;
      const int c = (slot % BROW) ^ (HB ? swz_kn_h(k) : swz_kn(k));
      // N % BV == 0: a chunk is inside the row or wholly past it.
      const int col = EDGE ? min(n0 + BV * c, N - BV) - n0 : BV * c;
      b_off[j] = static_cast<unsigned>(k * N + col) * static_cast<unsigned>(sizeof(BT));
    }
  }
  const long long a_len = static_cast<long long>(M) * K;
  const long long b_len = static_cast<long long>(N) * K;
  auto fetch = [&](float* as, BT* bs, int kt) {
    const int k0 = kt * BK;
    const long long a0 = static_cast<long long>(m0) * K + k0;
    const long long b0 = BNK ? static_cast<long long>(n0) * K + k0 : static_cast<long long>(k0) * N + n0;
    const unsigned a_bytes = bytes_left<float>(a_len, a0);
    const unsigned b_bytes = bytes_left<BT>(b_len, b0);
#pragma unroll
    for (int j = 0; j < A_INST; ++j)
      lds_buf16(A + a0, a_bytes, a_off[j], as + 4 * (C::kWaves * j + wave) * 64);
#pragma unroll
    for (int j = 0; j < B_INST; ++j)
      lds_buf16(B + b0, b_bytes, b_off[j], bs + BV * (C::kWaves * j + wave) * 64);
  };

#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[mb][nb][v] = 0.0f;

  // Fragments of one quarter of a K tile (MFMA k-slices s = 4 q .. 4 q + 3):
  // lane (li, lg) holds A[row][16 lg + s] and B[16 lg + s][col].
  struct Quarter {
    floatx4 a[MB];
    float b[NB][4];
  };
  auto read_q = [&](const float* as, const BT* bs, int q, Quarter& f) {
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      const int r = wm * C::WM + mb * 32 + li;
      const int c = (lg * 4 + q) ^ swz_rows(r);
      f.a[mb] = *reinterpret_cast<const floatx4*>(as + 4 * (r * 8 + c));
    }
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      if constexpr (BNK && !HB) {
        const int r = wn * C::WN + nb * 32 + li;
        const int c = (lg * 4 + q) ^ swz_rows(r);
        const floatx4 v = *reinterpret_cast<const floatx4*>(bs + 4 * (r * 8 + c));
#pragma unroll
        for (int e = 0; e < 4; ++e) f.b[nb][e] = v[e];
      } else if constexpr (BNK) {
        // Row r holds k = 0..31 as 4 chunks of 8; this lane's k = 16 lg + 4 q + e
        // are halves 4 (q & 1) .. 4 (q & 1) + 3 of chunk 2 lg + q / 2.
        const int r = wn * C::WN + nb * 32 + li;
        const int c = (lg * 2 + (q >> 1)) ^ swz_rows_h(r);
        const _Float16* p = bs + 8 * (r * 4 + c) + 4 * (q & 1);
#pragma unroll
        for (int e = 0; e < 4; ++e) f.b[nb][e] = static_cast<float>(p[e]);
      } else {
        const int n = wn * C::WN + nb * 32 + li;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int k = lg * 16 + 4 * q + e;
          if constexpr (HB) {
            const int c = (n >> 3) ^ swz_kn_h(k);
            f.b[nb][e] = static_cast<float>(bs[8 * (k * BROW + c) + (n & 7)]);
          } else {
            const int c = (n >> 2) ^ swz_kn(k);
            f.b[nb][e] = bs[4 * (k * BROW + c) + (n & 3)];
          }
        }
      }
    }
  };
  auto mma_q = [&](const Quarter& f) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
          acc[mb][nb] = __builtin_amdgcn_mfma_f32_32x32x2f32(f.a[mb][e], f.b[nb][e], acc[mb][nb], 0, 0, 0);
      }
    }
  };

  // Software pipeline over quarters: each quarter's fragments are read while
  // the previous quarter's MFMAs run. The stage hand-over sits before a K
  // tile's last quarter: it waits for the direct loads of the next tile (S - 2
  // later tiles may stay in flight), makes every wave's loads of it visible
  // (so that tile's first quarter can be read during this tile's last), and
  // ends every wave's reads of the current stage, which the fetch after it
  // refills with the tile S steps ahead. That fetch and the read after the
  // barrier are unconditional so that nothing splits the block: near the end
  // the fetch loads tile kt1 - 1 again into a finished stage and the read
  // takes a stale quarter that is never used. Scheduling barriers keep each
  // quarter's reads ahead of the previous quarter's MFMAs.
  auto pin = [] {
#if defined(__HIP_DEVICE_COMPILE__)
    __builtin_amdgcn_sched_group_barrier(0x100, 16, 0);  // DS reads
    __builtin_amdgcn_sched_group_barrier(0x008, 16, 0);  // MFMAs
    __builtin_amdgcn_sched_barrier(0);
#endif
  };
  // After the stage barrier every wave of the workgroup resumes at once (the
  // two on each SIMD, on 256 x 128 tiles): two MFMAs go first, then each of
  // the fetch's loads, with its address arithmetic, behind one more MFMA, so
  // the matrix core stays busy while they issue (4096^3: 947 us with the
  // loads first, 921 us interleaved).
  auto pin_after_barrier = [] {
#if defined(__HIP_DEVICE_COMPILE__)
    __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);  // MFMAs
#pragma unroll
    for (int i = 0; i < kLoads; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // a VMEM read (the fetch)
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // an MFMA
    }
    __builtin_amdgcn_sched_group_barrier(0x100, 16, 0);  // DS reads
    __builtin_amdgcn_sched_group_barrier(0x008, 16, 0);  // the remaining MFMAs
    __builtin_amdgcn_sched_barrier(0);
#endif
  };
  Quarter x, y;
  auto tile = [&](auto st, int kt) {
    constexpr int cur = decltype(st)::value;
    using Next = std::integral_constant<int, (cur + 1) % S>;
    const float* as = a_stage(st);
    const BT* bs = b_stage(st);
    read_q(as, bs, 1, y);
    mma_q(x);
    pin();
    read_q(as, bs, 2, x);
    mma_q(y);
    pin();
    read_q(as, bs, 3, y);
    mma_q(x);
    pin();
    stage_barrier<(S - 2) * kLoads>();
    fetch(a_stage(st), b_stage(st), min(kt + S, kt1 - 1));
    read_q(a_stage(Next{}), b_stage(Next{}), 0, x);
    mma_q(y);
    pin_after_barrier();
  };
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  using I2 = std::integral_constant<int, 2>;

  fetch(As0, Bs0, kt0);
  fetch(As1, Bs1, min(kt0 + 1, kt1 - 1));
  if constexpr (S > 2) fetch(As2, Bs2, min(kt0 + 2, kt1 - 1));
  stage_barrier<(S - 1) * kLoads>();
  read_q(As0, Bs0, 0, x);
  int kt = kt0;
  for (; kt + S - 1 < kt1; kt += S) {
    tile(I0{}, kt);
    tile(I1{}, kt + 1);
    if constexpr (S > 2) tile(I2{}, kt + 2);
  }
  if (kt < kt1) tile(I0{}, kt);
  if constexpr (S > 2) {
    if (kt + 1 < kt1) tile(I1{}, kt + 1);
  }
  wait_all_memory();
  __syncthreads();
}

// Stores a tile's accumulators: element (r, c) of the tile to out[r * ld + c]
// (out at the tile's first element), rows < rows_left and columns < cols_left
// only (EDGE).
template <int BM, int BN, bool EDGE>
__device__ __forceinline__ void store_acc(const TileAcc<BM, BN>& acc, float* __restrict__ out,
                                          long long ld, int rows_left, int cols_left) {
  using C = TileCfg<BM, BN>;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int li = lane & 31;
  const int lg = lane >> 5;
  const int wm = wave / C::WGN;
  const int wn = wave % C::WGN;
#if defined(__HIP_DEVICE_COMPILE__)
  // In the stream-K kernel's tile loop the per-element offsets row ld + col
  // are loop-invariant; hoisted they held registers through the K loop (36
  // bytes of spills at 128 x 128). An opaque ld keeps them here.
  asm volatile("" : "+s"(ld));
#endif
#pragma unroll
  for (int mb = 0; mb < C::MB; ++mb) {
#pragma unroll
    for (int nb = 0; nb < C::NB; ++nb) {
      const int col = wn * C::WN + nb * 32 + li;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int row = wm * C::WM + mb * 32 + 8 * (v >> 2) + 4 * lg + (v & 3);
        if (!EDGE || (row < rows_left && col < cols_left)) out[row * ld + col] = acc[mb][nb][v];
      }
    }
  }
}

template <int BM, int BN, bool BNK, typename BT = float, bool EDGE = false>
__global__ __launch_bounds__((TileCfg<BM, BN>::kThreads), (TileCfg<BM, BN>::kMinBlocks)) void
gemm_f32_mfma_dma_kernel(const float* __restrict__ A, const BT* __restrict__ B,
                         float* __restrict__ C, int M, int N, int K, int tiles_m, int tiles_n) {
  int tm, tn;
  tile_of(blockIdx.x, tiles_m, tiles_n, tm, tn);
  const int m0 = tm * BM;
  const int n0 = tn * BN;
  TileAcc<BM, BN> acc;
  dma_tile<BM, BN, BNK, BT, EDGE>(A, B, M, N, K, m0, n0, 0, K / BK, acc);
  store_acc<BM, BN, EDGE>(acc, C + static_cast<long long>(m0) * N + n0, N, M - m0, N - n0);
}

// Stream-K tail (full tiles only): T tiles, of which the first `dp` in
// tile_of order are computed whole by workgroups 0 .. dp - 1 (one round of
// one per CU), and the remaining T - dp tiles' k-iterations are split evenly
// over the workgroups dp .. dp + nsk - 1 (nsk = min(dp, I): none is empty):
// workgroup dp + s takes iterations [s I / nsk, (s + 1) I / nsk) of the
// tail's I = (T - dp) nk, tile by tile.
// Running beside the data-parallel round (two workgroups per CU), every CU
// then does the same work whatever T is (512 x 11008 x 4096: 344 tiles on
// 256 CUs). A tail tile one workgroup covers whole is stored to C; a split
// tile leaves one record per workgroup (slot 0 its first tile, slot 1 its
// last), which gemm_sk_fixup_kernel adds in workgroup order.
struct SkPlan {
  int dp = 0;        // data-parallel tiles (one per CU)
  int nsk = 0;       // stream-K workgroups
  int nk = 0;        // K tiles per output tile
  long long I = 0;   // tail iterations (tail tiles x nk)
};

__host__ __device__ inline long long sk_begin(long long s, const SkPlan& p) {
  return s * p.I / p.nsk;
}

// Stream-K workgroup whose range holds tail iteration it.
__device__ inline long long sk_worker(long long it, const SkPlan& p) {
  long long s = (it * p.nsk + p.nsk - 1) / p.I;
  if (s >= p.nsk) s = p.nsk - 1;
  while (s + 1 < p.nsk && sk_begin(s + 1, p) <= it) ++s;
  while (s > 0 && sk_begin(s, p) > it) --s;
  return s;
}

template <int BM, int BN, bool BNK, typename BT>
__global__ __launch_bounds__(kThreads, 2) void gemm_sk_kernel(
    const float* __restrict__ A, const BT* __restrict__ B, float* __restrict__ C,
    float* __restrict__ rec, int M, int N, int K, int tiles_m, int tiles_n, SkPlan plan) {
  TileAcc<BM, BN> acc;
  // One loop for both kinds of workgroup (a single inlined copy of the tile
  // loop): a data-parallel workgroup g covers iterations [0, nk) of tile g; a
  // stream-K workgroup its share of the tail, whose tile t is tile dp + t.
  const int g = blockIdx.x;
  const bool dp = g < plan.dp;
  const long long s = dp ? 0 : g - plan.dp;
  const long long i0 = dp ? 0 : sk_begin(s, plan);
  const long long i1 = dp ? plan.nk : sk_begin(s + 1, plan);
  const int first_tile = dp ? g : plan.dp;
  for (long long it = i0; it < i1;) {
    const long long t = it / plan.nk;
    const int ka = static_cast<int>(it - t * plan.nk);
    const long long tend = (t + 1) * plan.nk;
    const int kb = static_cast<int>((i1 < tend ? i1 : tend) - t * plan.nk);
    int tm, tn;
    tile_of(first_tile + static_cast<int>(t), tiles_m, tiles_n, tm, tn);
    const int m0 = tm * BM;
    const int n0 = tn * BN;
    dma_tile<BM, BN, BNK, BT, false>(A, B, M, N, K, m0, n0, ka, kb, acc);
    if (ka == 0 && kb == plan.nk) {
      store_acc<BM, BN, false>(acc, C + static_cast<long long>(m0) * N + n0, N, BM, BN);
    } else {
      const int slot = it == i0 ? 0 : 1;
      store_acc<BM, BN, false>(acc, rec + (s * 2 + slot) * static_cast<long long>(BM * BN), BN,
                               BM, BN);
    }
    it = t * plan.nk + kb;
  }
}

// Split tail tiles: C = the tile's records added in workgroup order. One
// block per (tail tile, 1024 elements); tiles one workgroup covered whole are
// skipped (already stored).
template <int BM, int BN, bool EDGE = false>
__global__ __launch_bounds__(256) void gemm_sk_fixup_kernel(const float* __restrict__ rec,
                                                            float* __restrict__ C, int M, int N,
                                                            int tiles_m, int tiles_n,
                                                            SkPlan plan) {
  const long long t = blockIdx.x;
  const long long sf = sk_worker(t * plan.nk, plan);
  const long long sl = sk_worker(t * plan.nk + plan.nk - 1, plan);
  if (sf == sl) return;
  // workgroups after sf start inside the tile (slot 0); sf only when it
  // starts exactly at the tile
  const int slot_f = sk_begin(sf, plan) == t * plan.nk ? 0 : 1;
  const int e = 4 * (static_cast<int>(blockIdx.y) * 256 + static_cast<int>(threadIdx.x));
  floatx4 v = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
  // (unrolled so a group's loads are in flight together; the adds keep
  // workgroup order)
#pragma unroll 8
  for (long long s = sf; s <= sl; ++s) {
    const long long r = s * 2 + (s == sf ? slot_f : 0);
    v += *reinterpret_cast<const floatx4*>(rec + r * static_cast<long long>(BM * BN) + e);
  }
  int tm, tn;
  tile_of(plan.dp + static_cast<int>(t), tiles_m, tiles_n, tm, tn);
  const int row = tm * BM + e / BN;
  const int col = tn * BN + e % BN;
  float* dst = C + static_cast<long long>(row) * N + col;
  if constexpr (!EDGE) {
    *reinterpret_cast<floatx4*>(dst) = v;
  } else if (row < M) {
#pragma unroll
    for (int q = 0; q < 4; ++q)
      if (col + q < N) dst[q] = v[q];
  }
}

// The direct-load kernel can be switched off (ENGINE_GEMM_NO_DMA=1) to
// compare it with the register-staged kernel on the same shapes.
bool dma_enabled() {
  static const bool on = [] {
    const char* v = std::getenv("ENGINE_GEMM_NO_DMA");
    return !(v != nullptr && v[0] == '1');
  }();
  return on;
}

// Direct loads need K % BK == 0, 16-byte aligned operands and 16-byte
// aligned B rows ([K x N] rows of N elements; [N x K] rows of K), and every
// lane's byte offset from a tile's corner (up to BM rows of A, BN rows of an
// [N x K] B or BK rows of a [K x N] B) must fit the 31 bits of a buffer
// load's offset.
template <int BM, int BN, typename BT, bool BNK>
bool direct_ok(const GemmArgs& a) {
  constexpr long long kBVec = 16 / static_cast<long long>(sizeof(BT));
  constexpr long long kLim = 0x7fffffffLL;
  const long long b_span = BNK ? static_cast<long long>(BN) * a.K : static_cast<long long>(BK) * a.N;
  return dma_enabled() && a.K % BK == 0 && aligned_to(a.A, 16) && aligned_to(a.B, 16) &&
         (BNK || a.N % kBVec == 0) && static_cast<long long>(BM) * a.K * 4 <= kLim &&
         b_span * static_cast<long long>(sizeof(BT)) <= kLim;
}

// The 256 x 128 tile can be switched off (ENGINE_GEMM_NO_BIG=1) to compare
// it with 128 x 128 on the same shapes.
bool big_tile_enabled() {
  static const bool on = [] {
    const char* v = std::getenv("ENGINE_GEMM_NO_BIG");
    return !(v != nullptr && v[0] == '1');
  }();
  return on;
}

template <int BM, int BN, typename BT, bool BNK>
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
  if (direct_ok<BM, BN, BT, BNK>(a)) {
    // Whole tiles take the plain kernel, ragged M / N its EDGE form.
    constexpr int kDmaThreads = TileCfg<BM, BN>::kThreads;
    if (M % BM == 0 && N % BN == 0) {
      gemm_f32_mfma_dma_kernel<BM, BN, BNK, BT, false><<<grid, kDmaThreads, 0, stream>>>(
          a.A, B, a.C, M, N, K, tiles_m, tiles_n);
    } else {
      gemm_f32_mfma_dma_kernel<BM, BN, BNK, BT, true><<<grid, kDmaThreads, 0, stream>>>(
          a.A, B, a.C, M, N, K, tiles_m, tiles_n);
    }
    ENG_LAUNCH_CHECK();
    return;
  }
  if constexpr (TileCfg<BM, BN>::kBig) {
    // big_tile() only picks 256 x 128 when the direct loads apply
    ENG_CHECK(false, "matmul: 256-row tiles need the direct-load kernel");
  } else {
#define ENG_GEMM_LAUNCH(VA_, VB_)                                                    \
    gemm_f32_mfma_kernel<BM, BN, BT, BNK, VA_, VB_><<<grid, kThreads, 0, stream>>>( \
        a.A, B, a.C, M, N, K, tiles_m, tiles_n)
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
}

// Tile shape: the largest of 128 x 128, 128 x 64, 64 x 64 whose makespan (rounds
// of one tile per CU, times the tile's share of the work) is not worse than a
// smaller shape's. Smaller tiles re-read A and B more, so ties go to the larger
// -- except that 64 x 64 wins a tie with 128 x 64 when 128 x 64 leaves at most
// one workgroup per CU: two co-resident 64 x 64 workgroups hide each other's
// latency (MI355X: 512 x 4096 x 11008 361 vs 376 us, 512 x 4096 x 4096 138 vs
// 142 us). The same preference measured slower one step up (1024 x 4096 x 4096:
// 256 tiles of 128 x 128 258 us, 512 of 128 x 64 272 us) and with more than one
// workgroup per CU (512 x 11008 x 4096: 128 x 64 411 us, 64 x 64 420 us).
enum class Tile { T128x128, T128x64, T64x64 };

Tile choose_tile(long long M, long long N) {
  const long long cus = device_cu_count();
  auto tiles = [&](long long bm, long long bn) { return ((M + bm - 1) / bm) * ((N + bn - 1) / bn); };
  auto makespan = [&](long long bm, long long bn) {
    const long long rounds = (tiles(bm, bn) + cus - 1) / cus;
    return static_cast<double>(rounds) * static_cast<double>(bm * bn) / (128.0 * 128.0);
  };
  const double t1 = makespan(128, 128);
  const double t2 = makespan(128, 64);
  const double t3 = makespan(64, 64);
  if (t1 <= t2 && t1 <= t3) return Tile::T128x128;
  if (t2 < t3 || (t2 == t3 && tiles(128, 64) > cus)) return Tile::T128x64;
  return Tile::T64x64;
}

// Stream-K tail for 128 x 128 tiles when their count T falls between one
// and two rounds of one tile per CU (CUs < T < 2 CUs; every other shape
// keeps choose_tile's tiling): full tiles and the direct-load conditions
// only. ENGINE_GEMM_NO_SK=1 switches it off.
// The single-launch small-GEMM kernel can be switched off
// (ENGINE_GEMM_NO_SMALL=1).
bool small_enabled() {
  static const bool on = [] {
    const char* v = std::getenv("ENGINE_GEMM_NO_SMALL");
    return !(v != nullptr && v[0] == '1');
  }();
  return on;
}

bool sk_enabled() {
  static const bool on = [] {
    const char* v = std::getenv("ENGINE_GEMM_NO_SK");
    return !(v != nullptr && v[0] == '1');
  }();
  return on;
}

template <typename BT, bool BNK>
bool run_gemm_sk(const GemmArgs& a, hipStream_t stream) {
  constexpr int BM = 128, BN = 128;
  if (!sk_enabled() || !direct_ok<BM, BN, BT, BNK>(a)) return false;
  if (a.M % BM != 0 || a.N % BN != 0 || a.K / BK < 8) return false;
  const long long cus = device_cu_count();
  const int tiles_m = static_cast<int>(a.M / BM);
  const int tiles_n = static_cast<int>(a.N / BN);
  const long long T = static_cast<long long>(tiles_m) * tiles_n;
  if (T <= cus || T >= 2 * cus) return false;
  SkPlan plan;
  plan.dp = static_cast<int>(cus);
  plan.nk = static_cast<int>(a.K / BK);
  plan.I = (T - cus) * plan.nk;
  plan.nsk = static_cast<int>(std::min<long long>(plan.dp, plan.I));
  StreamScratch records(stream, static_cast<std::size_t>(plan.nsk) * 2 * BM * BN * sizeof(float), 2);
  float* rec = static_cast<float*>(records.get());
  const BT* B = static_cast<const BT*>(a.B);
  const int M = static_cast<int>(a.M), N = static_cast<int>(a.N), K = static_cast<int>(a.K);
  gemm_sk_kernel<BM, BN, BNK, BT><<<static_cast<unsigned>(plan.dp + plan.nsk), kThreads, 0, stream>>>(
      a.A, B, a.C, rec, M, N, K, tiles_m, tiles_n, plan);
  ENG_LAUNCH_CHECK();
  gemm_sk_fixup_kernel<BM, BN><<<dim3(static_cast<unsigned>(T - cus), BM * BN / 1024), 256, 0,
                                 stream>>>(rec, a.C, M, N, tiles_m, tiles_n, plan);
  ENG_LAUNCH_CHECK();
  return true;
}

// Small GEMMs in one launch: one 32 x 32 tile of C per workgroup, its four
// waves each taking a quarter of K straight from global memory into the
// v_mfma_f32_32x32x2_f32 operands, the four partial tiles summed through LDS
// in wave order (512^3: 256 workgroups, every SIMD of the chip busy, where
// 64 x 64 tiles keep a quarter of the CUs). MFMA step t of a lane group g
// takes k = k8 + 4 g + t (k8 a multiple of 8): lane (r, g) loads A[row r][k8
// + 4 g .. + 3] as one float4 and B[k8 + 4 g + t][column r] as four floats
// (32 lanes read 128 consecutive bytes of a B row). Loads run DS iterations
// of 8 k ahead in a register ring; two accumulators (even and odd t) per
// wave, added before the wave sum. Needs M and N multiples of 32, K of 256,
// A rows 16-byte aligned, B row-major [K x N].
namespace small {
constexpr int DS = 8;  // iterations (8 k each) in flight per wave
}
__global__ __launch_bounds__(256) void gemm_small_splitk_kernel(const float* __restrict__ A,
                                                               const float* __restrict__ B,
                                                               float* __restrict__ C, int M, int N,
                                                               int K, int tiles_n) {
  constexpr int D = small::DS;
  __shared__ float red[4][16][64];
  const int tm = blockIdx.x / tiles_n;
  const int tn = blockIdx.x % tiles_n;
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int r = lane & 31;
  const int g = lane >> 5;
  const int kq = K / 4;
  const int iters = kq / 8;  // a multiple of D (K % 256 == 0)
  const float* ap = A + static_cast<long long>(tm * 32 + r) * K + wave * kq + 4 * g;
  const float* bp = B + static_cast<long long>(wave * kq + 4 * g) * N + tn * 32 + r;
  const long long bstep = 8LL * N;
  floatx4 a[D];
  float b[D][4];
  auto load = [&](int d, int it) {
    a[d] = *reinterpret_cast<const floatx4*>(ap + 8 * it);
    const float* q = bp + it * bstep;
#pragma unroll
    for (int t = 0; t < 4; ++t) b[d][t] = q[static_cast<long long>(t) * N];
  };
#pragma unroll
  for (int d = 0; d < D; ++d) load(d, d);
  floatx16 acc0, acc1;
#pragma unroll
  for (int v = 0; v < 16; ++v) acc0[v] = acc1[v] = 0.0f;
  for (int i = 0; i < iters; i += D) {
#pragma unroll
    for (int d = 0; d < D; ++d) {
      acc0 = __builtin_amdgcn_mfma_f32_32x32x2f32(a[d][0], b[d][0], acc0, 0, 0, 0);
      acc1 = __builtin_amdgcn_mfma_f32_32x32x2f32(a[d][1], b[d][1], acc1, 0, 0, 0);
      acc0 = __builtin_amdgcn_mfma_f32_32x32x2f32(a[d][2], b[d][2], acc0, 0, 0, 0);
      acc1 = __builtin_amdgcn_mfma_f32_32x32x2f32(a[d][3], b[d][3], acc1, 0, 0, 0);
      if (i + D + d < iters) load(d, i + D + d);
    }
  }
#pragma unroll
  for (int v = 0; v < 16; ++v) red[wave][v][lane] = acc0[v] + acc1[v];
  __syncthreads();
  // Accumulator element v of lane l: C[8 (v / 4) + 4 (l / 32) + v % 4][l % 32].
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int idx = threadIdx.x + 256 * q;
    const int v = idx >> 6;
    const int l = idx & 63;
    const float sum = ((red[0][v][l] + red[1][v][l]) + red[2][v][l]) + red[3][v][l];
    const int row = tm * 32 + 8 * (v >> 2) + 4 * (l >> 5) + (v & 3);
    const int col = tn * 32 + (l & 31);
    C[static_cast<long long>(row) * N + col] = sum;
  }
}

template <typename BT, bool BNK>
bool run_gemm_small(const GemmArgs& a, hipStream_t stream) {
  if constexpr (BNK || !std::is_same<BT, float>::value) {
    return false;
  } else {
    if (!small_enabled() || a.M % 32 != 0 || a.N % 32 != 0 || a.K % 256 != 0 ||
        !aligned_to(a.A, 16))
      return false;
    const long long cus = device_cu_count();
    if (2 * (a.M / 64) * (a.N / 64) > cus) return false;  // 64 x 64 tiles fill half the CUs
    const long long tiles = (a.M / 32) * (a.N / 32);
    ENG_CHECK(tiles <= 0x7fffffffLL, "matmul: too many tiles for one launch");
    gemm_small_splitk_kernel<<<static_cast<unsigned>(tiles), 256, 0, stream>>>(
        a.A, static_cast<const float*>(a.B), a.C, static_cast<int>(a.M), static_cast<int>(a.N),
        static_cast<int>(a.K), static_cast<int>(a.N / 32));
    ENG_LAUNCH_CHECK();
    return true;
  }
}

// 256 x 128 tiles where choose_tile's model takes 128 x 128 and gives the
// larger tile no longer a makespan (rounds of one tile per CU, times the
// tile's area: 4096^3 has 512 such tiles against 1024, two rounds of twice
// the work against four), and the direct loads apply.
template <typename BT, bool BNK>
bool big_tile(const GemmArgs& a) {
  if (!big_tile_enabled() || !direct_ok<256, 128, BT, BNK>(a)) return false;
  if (choose_tile(a.M, a.N) != Tile::T128x128) return false;
  const long long cus = device_cu_count();
  auto rounds = [&](long long bm, long long bn) {
    return (((a.M + bm - 1) / bm) * ((a.N + bn - 1) / bn) + cus - 1) / cus;
  };
  return 2 * rounds(256, 128) <= rounds(128, 128);
}

template <typename BT, bool BNK>
void run_gemm_tiled(const GemmArgs& a, hipStream_t stream) {
  if (run_gemm_sk<BT, BNK>(a, stream)) return;
  if (run_gemm_small<BT, BNK>(a, stream)) return;
  if (big_tile<BT, BNK>(a)) {
    run_gemm<256, 128, BT, BNK>(a, stream);
    return;
  }
  switch (choose_tile(a.M, a.N)) {
    case Tile::T128x128:
      run_gemm<128, 128, BT, BNK>(a, stream);
      break;
    case Tile::T128x64:
      run_gemm<128, 64, BT, BNK>(a, stream);
      break;
    case Tile::T64x64:
      run_gemm<64, 64, BT, BNK>(a, stream);
      break;
  }
}

// ---------------------------------------------------------------------------
// fp16 weights on the fp16 matrix cores: C[M x N] = diag(rscale) (P0 + P1 +
// P2) . W for fp16 weights W, given [N x K] (output-major: the kernel reads
// W^T) or [K x N] (the reference layout), and the three fp16 planes P of the
// scaled activation rows (launch_rmsnorm_split3). Every product of an fp16
// plane value and an fp16 weight is exact in fp32 and the planes sum to the
// scaled row (to 2^-39 of its largest value), so this is the FP32 GEMM's
// arithmetic on v_mfma_f32_32x32x16_f16, which runs 16 times the FP32
// instruction's rate: three of them (one per plane) per 32 x 32 x 16 block
// against eight v_mfma_f32_32x32x2_f32.
//
// Tiles of 128 x 128 (8 waves, 4 x 2, of 32 x 64: per 16-deep slice three
// plane fragments and two weight fragments feed six MFMAs; four LDS stages
// of 32 KiB) or, from 60% of a round of them up, 128 x 256 (8 waves, 2 x 4,
// of 64 x 64; three stages of 40 KiB): K step 32 (two slices), one workgroup
// per CU. The planes are K-blocked (launch_rmsnorm_split3), so a plane tile
// of one K step is 8 KiB in one piece and every load instruction reads whole
// cache lines; with the planes row-major each instruction touched 16 rows of
// 64 bytes, half of each 128-byte line, and the vector memory path, not the
// MFMAs, set the pace. Operand layout of the instruction (checked on the
// device): A[i][k] in lane i + 32 (k / 8) element k % 8, B[k][j] in lane j +
// 32 (k / 8) element k % 8, the accumulator as for the FP32 instruction.
// Plane fragments, and [N x K] weight fragments, are one 16-byte LDS read of
// their row (tiles are rows of 4 16-byte chunks, chunk c of row r at c ^
// swz_rows_h(r)); [K x N] weight fragments are two transposing reads of the
// k rows. Direct loads, the slice read-ahead, the stage hand-over and the
// interleaved fetch follow the FP32 kernel. Past one round of tiles a last
// round at most half full, and below half a round every tile, is split by K
// (gemm_h3_sk_kernel, the plan of gemm_sk_kernel).
namespace h3 {
// Tiles of BMT x BNT: 128 x 128 and 128 x 256 on 8 waves, 64 x 128 on 4 waves
// (two workgroups per CU). BNT / 64 waves along N and the rest along M, each
// wave a WM x 64 block as MB x 2 32 x 32 MFMA blocks; every shape loads its
// three plane tiles with three direct loads per thread and K step.
template <int BMT, int BNT>
struct Shape {
  static_assert((BMT == 128 && (BNT == 128 || BNT == 256)) || (BMT == 64 && BNT == 128),
                "tile shape");
  static constexpr int BM = BMT;
  static constexpr int WAVES = BMT / 16;
  static constexpr int THREADS = 64 * WAVES;
  static constexpr int PT = BM * BK;                   // halves of one plane tile
  static constexpr int A_INST = 3 * PT / 8 / THREADS;  // direct loads per thread per K step (A planes)
  static constexpr int WGN = BNT / 64;
  static constexpr int WM = BM / (WAVES / WGN);
  static constexpr int WN = 64;
  static constexpr int MB = WM / 32;
  static constexpr int NB = WN / 32;
  static constexpr int B_INST = BNT * BK / 8 / THREADS;  // direct loads per thread per K step (B)
  static constexpr int LOADS = A_INST + B_INST;
  static constexpr int PER_CU = BMT == 64 ? 2 : 1;       // workgroups a CU runs at once
  static_assert(A_INST == 3 && B_INST * THREADS * 8 == BNT * BK && MB >= 1, "tile shape");
  static_assert(THREADS == 4 * BMT && PER_CU == (BMT == 64 ? 2 : 1), "the kernels' launch bounds");
};
template <int BMT, int BNT>
using Acc = floatx16[Shape<BMT, BNT>::MB][Shape<BMT, BNT>::NB];
constexpr int BM_MAX = 128;  // tallest tile (the offset bounds of gemm_h3_applies)
}  // namespace h3

// Reference-layout B tiles ([K x N] rows of BNT halves, 16-byte chunks):
// chunk c of row k sits at c ^ swz_h3_kn(k). A transposing read touches 8 rows
// (4 consecutive, and the 4 eight rows on) x 64 bytes (4 chunks from a
// multiple of 4); the swizzle puts 4 consecutive rows' chunk groups on 4
// distinct 64-byte bank slots.
__device__ __forceinline__ int swz_h3_kn(int k) { return 4 * (k & 3); }

// K tiles [kt0, kt1) of the BMT x BNT tile at (m0, n0) into acc (zeroed
// here); ends with a barrier, so a following call may refill the stages. BKN:
// B given [K x N] (the reference layout) instead of [N x K].
template <int S, int BMT, int BNT, bool BKN, bool EDGE>
__device__ __forceinline__ void h3_tile(const _Float16* __restrict__ P,
                                        const _Float16* __restrict__ B, int M, int N, int K,
                                        int m0, int n0, int kt0, int kt1,
                                        h3::Acc<BMT, BNT>& acc) {
  using Sh = h3::Shape<BMT, BNT>;
  static_assert(S >= 3 && S <= 4, "stages");
  constexpr int THREADS = Sh::THREADS;
  constexpr int PT = Sh::PT;
  constexpr int WGN = Sh::WGN;
  constexpr int WM = Sh::WM;
  constexpr int WN = Sh::WN;
  constexpr int MB = Sh::MB;
  constexpr int NB = Sh::NB;
  constexpr int B_INST = Sh::B_INST;
  constexpr int LOADS = Sh::LOADS;
  constexpr int AT = 3 * PT;    // halves of a stage's plane tiles
  constexpr int BTL = BNT * BK; // halves of a stage's B tile
  typedef _Float16 halfx8v __attribute__((ext_vector_type(8)));
  typedef _Float16 halfx4v __attribute__((ext_vector_type(4)));
  typedef short shortx4v __attribute__((ext_vector_type(4)));
  __shared__ __attribute__((aligned(1024))) _Float16 As0[AT];
  __shared__ __attribute__((aligned(1024))) _Float16 As1[AT];
  __shared__ __attribute__((aligned(1024))) _Float16 As2[AT];
  __shared__ __attribute__((aligned(1024))) _Float16 As3[S > 3 ? AT : 8];
  __shared__ __attribute__((aligned(1024))) _Float16 Bs0[BTL];
  __shared__ __attribute__((aligned(1024))) _Float16 Bs1[BTL];
  __shared__ __attribute__((aligned(1024))) _Float16 Bs2[BTL];
  __shared__ __attribute__((aligned(1024))) _Float16 Bs3[S > 3 ? BTL : 8];
  auto a_stage = [&](auto st) -> _Float16* {
    if constexpr (decltype(st)::value == 0) return As0;
    else if constexpr (decltype(st)::value == 1) return As1;
    else if constexpr (decltype(st)::value == 2) return As2;
    else return As3;
  };
  auto b_stage = [&](auto st) -> _Float16* {
    if constexpr (decltype(st)::value == 0) return Bs0;
    else if constexpr (decltype(st)::value == 1) return Bs1;
    else if constexpr (decltype(st)::value == 2) return Bs2;
    else return Bs3;
  };

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int li = lane & 31;
  const int lg = lane >> 5;
  const int wm = wave / WGN;
  const int wn = wave % WGN;

  // Direct loads: each load of wave w fills 16-byte slots 64 w + lane of a
  // THREADS-slot part of a tile (the three plane tiles, one part each; the B
  // tile's B_INST parts, part i holding slots THREADS i ..). In plane tiles and [N x K] B
  // tiles slot q is row q / 4, position q % 4, holding chunk (q % 4) ^
  // swz_rows_h(row) ([K x N] B tiles below). The planes are K-blocked
  // ([K / 32][M][32] each): a plane tile is a contiguous run of 64-byte rows,
  // so a load instruction covers 1 KiB in one piece (whole cache lines).
  [[maybe_unused]] unsigned a_off;  // (read by device code only)
  [[maybe_unused]] unsigned b_off[B_INST];
  {
    const int q = wave * 64 + lane;
    const int r = q >> 2;
    const int c = (q & 3) ^ swz_rows_h(r);
    const int ra = EDGE ? min(m0 + r, M - 1) - m0 : r;
    a_off = static_cast<unsigned>(ra * BK + 8 * c) * 2u;
  }
#pragma unroll
  for (int i = 0; i < B_INST; ++i) {
    const int q = i * THREADS + wave * 64 + lane;
    if constexpr (BKN) {
      // [K x N]: slot q is row q / CPR (one k), position q % CPR of its BNT / 8
      // chunks, holding chunk (q % CPR) ^ swz_h3_kn(row); chunks past N read
      // the tile's first (N % 8 == 0: a chunk is all in or all out).
      constexpr int CPR = BNT / 8;
      const int r = q / CPR;
      const int c = (q % CPR) ^ swz_h3_kn(r);
      const int cn = (!EDGE || n0 + 8 * c < N) ? 8 * c : 0;
      b_off[i] = static_cast<unsigned>(r * N + cn) * 2u;
    } else {
      const int r = q >> 2;
      const int c = (q & 3) ^ swz_rows_h(r);
      const int rb = EDGE ? min(n0 + r, N - 1) - n0 : r;
      b_off[i] = static_cast<unsigned>(rb * K + 8 * c) * 2u;
    }
  }
  // One buffer descriptor per plane (its whole extent) and one for the
  // tile's B (from its first element to the end of B, capped at 4 GiB), made
  // once; a K step moves only the scalar offset: (kt M + m0) 64 bytes into a
  // plane (under 2^31: M K 2 bytes is), kt 64 bytes along B's rows ([N x K])
  // or kt 32 N 2 bytes down them ([K x N]: under 2^31, K N 2 bytes is).
  // Rebuilding the descriptors per K step (64-bit adds, the range clamp)
  // took some 40 scalar instructions per wave and K step, issue slots the
  // MFMAs then waited behind.
  [[maybe_unused]] const long long plane = static_cast<long long>(M) * K;
  [[maybe_unused]] const long long b_first = BKN ? n0 : static_cast<long long>(n0) * K;
  [[maybe_unused]] const int b_step = BKN ? BK * N * 2 : BK * 2;
#if defined(__HIP_DEVICE_COMPILE__)
  const auto ra0 = __builtin_amdgcn_make_buffer_rsrc(const_cast<_Float16*>(P), 0,
                                                     static_cast<int>(plane * 2), kRsrcWord3);
  const auto ra1 = __builtin_amdgcn_make_buffer_rsrc(const_cast<_Float16*>(P + plane), 0,
                                                     static_cast<int>(plane * 2), kRsrcWord3);
  const auto ra2 = __builtin_amdgcn_make_buffer_rsrc(const_cast<_Float16*>(P + 2 * plane), 0,
                                                     static_cast<int>(plane * 2), kRsrcWord3);
  const auto rb = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<_Float16*>(B + b_first), 0,
      static_cast<int>(bytes_left<_Float16>(static_cast<long long>(N) * K, b_first)), kRsrcWord3);
#endif
  auto fetch = [&](_Float16* as, _Float16* bs, int kt) {
#if defined(__HIP_DEVICE_COMPILE__)
    const int soff = (kt * M + m0) * (BK * 2);
    _Float16* dst = as + 8 * wave * 64;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(ra0, dst, 16, static_cast<int>(a_off), soff, 0, 0);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(ra1, dst + PT, 16, static_cast<int>(a_off), soff, 0,
                                             0);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(ra2, dst + 2 * PT, 16, static_cast<int>(a_off), soff,
                                             0, 0);
#pragma unroll
    for (int i = 0; i < B_INST; ++i)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rb, bs + 8 * (i * THREADS + wave * 64), 16,
                                               static_cast<int>(b_off[i]), kt * b_step, 0, 0);
#endif
  };

  struct Slice {
    halfx8v a[3][MB];
    halfx8v b[NB];
  };
  auto read_s = [&](const _Float16* as, const _Float16* bs, int sl, Slice& f) {
    const int cq = 2 * sl + lg;  // this lane's chunk: k = 16 sl + 8 lg .. + 7
#pragma unroll
    for (int p = 0; p < 3; ++p) {
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        const int r = wm * WM + mb * 32 + li;
        f.a[p][mb] = *reinterpret_cast<const halfx8v*>(as + p * PT + r * BK + 8 * (cq ^ swz_rows_h(r)));
      }
    }
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      if constexpr (BKN) {
        // Two transposing reads (ds_read_b64_tr_b16) per fragment: in each
        // 16-lane group lane l names 8 bytes (row k0 + l / 4, columns cb + 4 (l
        // % 4) .. + 3) and receives column cb + l of the 4 rows. Group G of the
        // wave takes columns 16 (G % 2) .. + 15 of the block and k half G / 2,
        // which is the B operand's lane j + 32 (k / 8), element k % 8.
        const int l = lane & 15;
        const int G = lane >> 4;
        const int col = wn * WN + nb * 32 + 16 * (G & 1) + 4 * (l & 3);  // first of the lane's 4
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int k = 16 * sl + 8 * (G >> 1) + 4 * h + (l >> 2);
          const int off = k * (BNT * 2) + (((col >> 3) ^ swz_h3_kn(k)) << 4) + ((col & 7) << 1);
          const halfx4v v = __builtin_bit_cast(
              halfx4v, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                           (__attribute__((address_space(3))) shortx4v*)(
                               (__attribute__((address_space(3))) char*)bs + off)));
#pragma unroll
          for (int e = 0; e < 4; ++e) f.b[nb][4 * h + e] = v[e];
        }
      } else {
        const int r = wn * WN + nb * 32 + li;
        f.b[nb] = *reinterpret_cast<const halfx8v*>(bs + r * BK + 8 * (cq ^ swz_rows_h(r)));
      }
    }
  };
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[mb][nb][v] = 0.0f;
  auto mma_s = [&](const Slice& f) {
#pragma unroll
    for (int p = 0; p < 3; ++p) {
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
          acc[mb][nb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(f.a[p][mb], f.b[nb], acc[mb][nb], 0,
                                                               0, 0);
    }
  };
  auto pin = [] {
#if defined(__HIP_DEVICE_COMPILE__)
    __builtin_amdgcn_sched_group_barrier(0x100, 16, 0);  // DS reads
    __builtin_amdgcn_sched_group_barrier(0x008, 16, 0);  // MFMAs
    __builtin_amdgcn_sched_barrier(0);
#endif
  };
  // After the stage barrier: one MFMA, the next slice's fragment reads
  // (six MFMAs ahead of their use: a slice has only six per wave, so reads
  // placed after the fetch would leave one MFMA to cover their latency),
  // then the fetch's loads one per MFMA.
  auto pin_after_barrier = [] {
#if defined(__HIP_DEVICE_COMPILE__)
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    __builtin_amdgcn_sched_group_barrier(0x100, 16, 0);
#pragma unroll
    for (int i = 0; i < LOADS; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, 16, 0);
    __builtin_amdgcn_sched_barrier(0);
#endif
  };

  // As the FP32 kernel: the hand-over before a K step's last slice waits for
  // the next tile (S - 2 later tiles stay in flight) and refills the current
  // stage with the tile S steps ahead (clamped to the last tile: a duplicate
  // load into a finished stage); the read after it takes the next tile's
  // first slice (stale past the last tile, never used).
  Slice x, y;
  auto tile = [&](auto st, int kt) {
    constexpr int cur = decltype(st)::value;
    using Next = std::integral_constant<int, (cur + 1) % S>;
    read_s(a_stage(st), b_stage(st), 1, y);
    mma_s(x);
    pin();
    stage_barrier<(S - 2) * LOADS>();
    fetch(a_stage(st), b_stage(st), min(kt + S, kt1 - 1));
    read_s(a_stage(Next{}), b_stage(Next{}), 0, x);
    mma_s(y);
    pin_after_barrier();
  };
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  using I2 = std::integral_constant<int, 2>;
  using I3 = std::integral_constant<int, 3>;

  fetch(As0, Bs0, kt0);
  fetch(As1, Bs1, min(kt0 + 1, kt1 - 1));
  fetch(As2, Bs2, min(kt0 + 2, kt1 - 1));
  if constexpr (S > 3) fetch(As3, Bs3, min(kt0 + 3, kt1 - 1));
  stage_barrier<(S - 1) * LOADS>();
  read_s(As0, Bs0, 0, x);
  int kt = kt0;
  for (; kt + S - 1 < kt1; kt += S) {
    tile(I0{}, kt);
    tile(I1{}, kt + 1);
    tile(I2{}, kt + 2);
    if constexpr (S > 3) tile(I3{}, kt + 3);
  }
  if (kt < kt1) tile(I0{}, kt);
  if (kt + 1 < kt1) tile(I1{}, kt + 1);
  if constexpr (S > 3) {
    if (kt + 2 < kt1) tile(I2{}, kt + 2);
  }
  wait_all_memory();
  __syncthreads();
}

// acc times the row's 2^-e into dst (row r, column c of the tile at dst[r ld
// + c]); GUARD keeps rows < rows_left and columns < cols_left. Rows past M
// (an edge tile's clamped rows) take row M - 1's scale.
template <int BMT, int BNT, bool GUARD>
__device__ __forceinline__ void h3_store(const h3::Acc<BMT, BNT>& acc, const float* __restrict__ rscale,
                                         int M, int m0, float* __restrict__ dst, long long ld,
                                         int rows_left, int cols_left) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int li = lane & 31;
  const int lg = lane >> 5;
  using Sh = h3::Shape<BMT, BNT>;
  const int wm = wave / Sh::WGN;
  const int wn = wave % Sh::WGN;
#if defined(__HIP_DEVICE_COMPILE__)
  // In the stream-K kernel's tile loop the per-element offsets r ld + col
  // are loop-invariant, and hoisted they held 32-64 registers for the whole
  // K loop (spilling the 128 x 256 form); an opaque ld keeps them here.
  asm volatile("" : "+s"(ld));
#endif

  // Accumulator element v of lane (li, lg): row 8 (v / 4) + 4 lg + v % 4 of
  // the block, column li.
#pragma unroll
  for (int mb = 0; mb < Sh::MB; ++mb) {
#pragma unroll
    for (int nb = 0; nb < Sh::NB; ++nb) {
      const int col = wn * Sh::WN + nb * 32 + li;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int r = wm * Sh::WM + mb * 32 + 8 * (v >> 2) + 4 * lg + (v & 3);
        if (!GUARD || (r < rows_left && col < cols_left))
          dst[r * ld + col] = acc[mb][nb][v] * rscale[min(m0 + r, M - 1)];
      }
    }
  }
}

template <int S, int BMT, int BNT, bool BKN, bool EDGE>
__global__ __launch_bounds__(4 * BMT, BMT == 64 ? 2 : 1) void gemm_h3_kernel(
    const _Float16* __restrict__ P, const float* __restrict__ rscale, const _Float16* __restrict__ B,
    float* __restrict__ C, int M, int N, int K, int tiles_m, int tiles_n) {
  int tm, tn;
  tile_of(blockIdx.x, tiles_m, tiles_n, tm, tn);
  const int m0 = tm * BMT;
  const int n0 = tn * BNT;
  h3::Acc<BMT, BNT> acc;
  h3_tile<S, BMT, BNT, BKN, EDGE>(P, B, M, N, K, m0, n0, 0, K / BK, acc);
  h3_store<BMT, BNT, EDGE>(acc, rscale, M, m0, C + static_cast<long long>(m0) * N + n0, N, M - m0,
                      N - n0);
}

// Stream-K form (the plan of gemm_sk_kernel): workgroups 0 .. dp - 1 compute
// tiles 0 .. dp - 1 whole (whole rounds of one tile per resident workgroup,
// two per CU for 64-row tiles), and the rest split the remaining tiles' K
// tiles evenly, at most one workgroup per CU after its
// data-parallel tiles; a split tile leaves one record per workgroup (scaled
// rows, slot 0 its first tile, slot 1 its last) for gemm_sk_fixup_kernel.
template <int S, int BMT, int BNT, bool BKN, bool EDGE>
__global__ __launch_bounds__(4 * BMT, BMT == 64 ? 2 : 1) void gemm_h3_sk_kernel(
    const _Float16* __restrict__ P, const float* __restrict__ rscale, const _Float16* __restrict__ B,
    float* __restrict__ C, float* __restrict__ rec, int M, int N, int K, int tiles_m, int tiles_n,
    SkPlan plan) {
  constexpr int BM = BMT, BN = BNT;
  h3::Acc<BMT, BNT> acc;
  const int g = blockIdx.x;
  const bool dp = g < plan.dp;
  const long long s = dp ? 0 : g - plan.dp;
  const long long i0 = dp ? 0 : sk_begin(s, plan);
  const long long i1 = dp ? plan.nk : sk_begin(s + 1, plan);
  const int first_tile = dp ? g : plan.dp;
  for (long long it = i0; it < i1;) {
    const long long t = it / plan.nk;
    const int ka = static_cast<int>(it - t * plan.nk);
    const long long tend = (t + 1) * plan.nk;
    const int kb = static_cast<int>((i1 < tend ? i1 : tend) - t * plan.nk);
    int tm, tn;
    tile_of(first_tile + static_cast<int>(t), tiles_m, tiles_n, tm, tn);
    const int m0 = tm * BM;
    const int n0 = tn * BN;
    h3_tile<S, BMT, BNT, BKN, EDGE>(P, B, M, N, K, m0, n0, ka, kb, acc);
    if (ka == 0 && kb == plan.nk) {
      h3_store<BMT, BNT, EDGE>(acc, rscale, M, m0, C + static_cast<long long>(m0) * N + n0, N, M - m0,
                          N - n0);
    } else {
      const int slot = it == i0 ? 0 : 1;
      h3_store<BMT, BNT, false>(acc, rscale, M, m0,
                           rec + (s * 2 + slot) * static_cast<long long>(BM * BN), BN, BM, BN);
    }
    it = t * plan.nk + kb;
  }
}

// The fp16-MFMA form of the fp16-weight GEMM can be switched off
// (ENGINE_GEMM_NO_H3=1) to compare it with the FP32 MFMA on converted weights.
// The 128 x 256 tiles can be switched off (ENGINE_GEMM_H3_NO_WIDE=1).
bool h3_wide_enabled() {
  static const bool on = [] {
    const char* v = std::getenv("ENGINE_GEMM_H3_NO_WIDE");
    return !(v != nullptr && v[0] == '1');
  }();
  return on;
}

// The 64 x 128 tiles for M <= 64 can be switched off (ENGINE_GEMM_H3_NO_SHORT=1).
bool h3_short_enabled() {
  static const bool on = [] {
    const char* v = std::getenv("ENGINE_GEMM_H3_NO_SHORT");
    return !(v != nullptr && v[0] == '1');
  }();
  return on;
}

bool h3_enabled() {
  static const bool on = [] {
    const char* v = std::getenv("ENGINE_GEMM_NO_H3");
    return !(v != nullptr && v[0] == '1');
  }();
  return on;
}

}  // namespace

bool gemm_h3_applies(std::int64_t M, std::int64_t N, std::int64_t K, const void* B, bool b_kn) {
  constexpr long long kLim = 0x7fffffffLL;
  // K % 32 == 0, 16-byte aligned B rows, every lane's byte offset from a
  // tile's corner (up to 128 rows of K halves) within a buffer load's 31 bits
  // and each activation plane (M K halves) within 31 bits of byte offset
  return h3_enabled() && M > 0 && N > 0 && K > 0 && K % BK == 0 && M <= kLim && N <= kLim &&
         K <= kLim && aligned_to(B, 16) && static_cast<long long>(h3::BM_MAX) * K * 2 <= kLim &&
         M * K * 2 <= kLim && (!b_kn || (N % 8 == 0 && K * N * 2 <= kLim));
}

void launch_gemm_h3(const GemmH3Args& a, hipStream_t stream) {
  ENG_CHECK(gemm_h3_applies(a.M, a.N, a.K, a.B, a.b_kn) && aligned_to(a.P, 16) && a.rscale != nullptr,
            "matmul (fp16 weights): shape or alignment not supported");
  const int M = static_cast<int>(a.M), N = static_cast<int>(a.N), K = static_cast<int>(a.K);
  const long long cus = device_cu_count();
  auto run = [&](auto bmt, auto bnt, auto stages) {
    constexpr int BMT = decltype(bmt)::value;
    constexpr int BNT = decltype(bnt)::value;
    constexpr int S = decltype(stages)::value;
    using Sh = h3::Shape<BMT, BNT>;
    const long long slots = cus * Sh::PER_CU;  // workgroups resident at once
    const int tiles_m = (M + BMT - 1) / BMT;
    const int tiles_n = (N + BNT - 1) / BNT;
    const long long ntiles = static_cast<long long>(tiles_m) * tiles_n;
    ENG_CHECK(ntiles <= 0x7fffffffLL, "matmul: too many tiles for one launch");
    const bool whole = M % BMT == 0 && N % BNT == 0;
    // Stream-K, with at least 8 K tiles per tile (a round: one tile per
    // resident workgroup, Sh::PER_CU per CU): past one round when the last
    // round is at most half full (512 x 11008 on 128 x
    // 128 tiles: 88 of 256, 148.7 -> 138.3 us; at 176 of 256 the records and
    // the fix-up pass cost more than the split saves), the tail's workgroups
    // running after the whole rounds; below half a round every tile is split
    // (65-128 x 11008, 86 tiles: 57-59 -> 45-52 us; at 172 tiles, 1.5 pieces
    // a tile, 70-72 -> 78-84 us, so those run whole). Each split workgroup
    // takes at least 8 K tiles, so a small tail is not spread one K tile per
    // CU (384 x 11008, 2 tail tiles, 136.5 -> 102.7 us: the fix-up had summed
    // 128 records per element).
    const int nk = K / BK;
    const long long tail = ntiles >= slots ? ntiles % slots : ntiles;
    const bool split = sk_enabled() && nk >= 8 && tail != 0 && 2 * tail <= slots;
    SkPlan plan;
    plan.dp = static_cast<int>(ntiles - tail);
    plan.nk = nk;
    plan.I = tail * nk;
    // At most one split workgroup per CU, also for the 64-row tiles (two per
    // CU: 64 x 11008 x 4096 44.8 against 40.9 us; 3/4 and 1/2 of the CUs 44.7
    // and 53.7; 64 x 4096 x 4096 26.0 against 23.5).
    plan.nsk = static_cast<int>(std::max<long long>(1, std::min<long long>(cus, plan.I / 8)));
    auto go = [&](auto kn, auto edge) {
      constexpr bool KN = decltype(kn)::value;
      constexpr bool E = decltype(edge)::value;
      if (!split) {
        gemm_h3_kernel<S, BMT, BNT, KN, E><<<static_cast<unsigned>(ntiles), Sh::THREADS, 0, stream>>>(
            a.P, a.rscale, a.B, a.C, M, N, K, tiles_m, tiles_n);
        ENG_LAUNCH_CHECK();
        return;
      }
      StreamScratch records(
          stream, static_cast<std::size_t>(plan.nsk) * 2 * BMT * BNT * sizeof(float), 2);
      float* rec = static_cast<float*>(records.get());
      gemm_h3_sk_kernel<S, BMT, BNT, KN, E><<<static_cast<unsigned>(plan.dp + plan.nsk), Sh::THREADS,
                                         0, stream>>>(a.P, a.rscale, a.B, a.C, rec, M, N, K,
                                                      tiles_m, tiles_n, plan);
      ENG_LAUNCH_CHECK();
      gemm_sk_fixup_kernel<BMT, BNT, E>
          <<<dim3(static_cast<unsigned>(tail), BMT * BNT / 1024), 256, 0, stream>>>(
              rec, a.C, M, N, tiles_m, tiles_n, plan);
      ENG_LAUNCH_CHECK();
    };
    using std::integral_constant;
    if (a.b_kn) {
      if (whole)
        go(integral_constant<bool, true>{}, integral_constant<bool, false>{});
      else
        go(integral_constant<bool, true>{}, integral_constant<bool, true>{});
    } else {
      if (whole)
        go(integral_constant<bool, false>{}, integral_constant<bool, false>{});
      else
        go(integral_constant<bool, false>{}, integral_constant<bool, true>{});
    }
  };
  // 128 x 256 tiles (waves of 64 x 64, three 40 KiB stages) once they fill at
  // least 60% of a round of one tile per CU: each plane tile loaded feeds
  // twice the MFMAs (x 11008 x 4096: 512 rows 141 -> 128 us, one round of 172
  // wide tiles against 344 narrow ones split past the first round; 1280 rows
  // 332 -> 291; 2048 rows 489 -> 445; 512 x 12288: 148 -> 137). Below that
  // the narrow tiles fill the CUs better (384 rows, 129 wide tiles: 106
  // against 111 us; 256 rows 72 against 85), and so they do between one and
  // two rounds of wide tiles when more than a quarter round would be split
  // (1024 x 11008, 344 wide tiles, 88 split: 260 against 244 us on 688
  // unsplit narrow ones). Else 128 x 128 (waves of 32 x 64, four 32 KiB
  // stages).
  const long long wide_tiles = static_cast<long long>((M + 127) / 128) * ((N + 255) / 256);
  const long long wide_tail = wide_tiles % cus;
  const bool wide_split_heavy = wide_tiles > cus && wide_tiles < 2 * cus && 4 * wide_tail > cus &&
                                2 * wide_tail <= cus;
  using std::integral_constant;
  // Up to 64 rows: 64 x 128 tiles (4 waves of 32 x 64, two workgroups per
  // CU, three 20 KiB stages): no MFMA work on padding rows past M. 33-64 x
  // 11008 x 4096: 47 -> 34-38 us (4096 x 4096: 28 -> 22-23.5); four stages
  // measured 0.5-1 us slower. From 65 rows the 128-row tiles are faster
  // (65 x 11008: 43.3 against 51.1 us).
  if (M <= 64 && h3_short_enabled())
    run(integral_constant<int, 64>{}, integral_constant<int, 128>{}, integral_constant<int, 3>{});
  else if (h3_wide_enabled() && 5 * wide_tiles >= 3 * cus && !wide_split_heavy)
    run(integral_constant<int, 128>{}, integral_constant<int, 256>{}, integral_constant<int, 3>{});
  else
    run(integral_constant<int, 128>{}, integral_constant<int, 128>{}, integral_constant<int, 4>{});
}

void launch_gemm(const GemmArgs& a, hipStream_t stream) {
  ENG_CHECK(a.M <= 0x7fffffffLL && a.N <= 0x7fffffffLL && a.K <= 0x7fffffffLL,
            "matmul: dimensions must fit in 31 bits");
  if (a.b == Elem::F32) {
    if (a.b_nk) {
      run_gemm_tiled<float, true>(a, stream);
    } else {
      run_gemm_tiled<float, false>(a, stream);
    }
  } else {
    if (a.b_nk) {
      run_gemm_tiled<_Float16, true>(a, stream);
    } else {
      run_gemm_tiled<_Float16, false>(a, stream);
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
    // A single row is a GEMV, out[N] = A[0][K] . B[K x N]; a few rows share
    // passes over B (the GEMM's 64-row tile would waste most of its work).
    eng::GemvArgs gv;
    gv.W = B;
    gv.w = eng::Elem::F32;
    gv.x = A;
    gv.y = C;
    gv.N = N;
    gv.K = K;
    if (M == 1) {
      eng::launch_gemv(gv, s);
      return;
    }
    // 5 to 64 rows: one pass over B on the matrix cores (the 64-row GEMM tile
    // would leave most CUs idle); 2 to 4 rows: GEMV passes, each row equal to
    // its single-row product.
    const eng::SkinnyArgs sk = eng::skinny_args(gv, M);
    if (eng::skinny_applies(sk)) {
      eng::launch_skinny(sk, s);
      return;
    }
    if (eng::launch_gemv_kn_rows(gv, M, s)) return;
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
