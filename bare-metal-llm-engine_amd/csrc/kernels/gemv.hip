// gemv.hip -- decode GEMV entry points and their launch configuration.
//
// Reference layout, out[N] = x[K] . W[K x N] (gemv, gemv_fp16, the fp16-weight
// overload, rmsnorm_linear at M == 1; reference kernels/gemv.cu,
// kernels/gemv_fp16.cu, kernels/rmsnorm_linear.cu): gemv_stream_kernel over
// 512-byte row segments. When the column slabs alone cannot fill the GPU the
// rows are split into chunks whose fp32 partial sums go to the stream's
// scratch arena and gemv_reduce_kernel combines them in chunk order. Two launches
// instead of a "last workgroup reduces" handshake: on gfx950 the agent-scope
// release/acquire that handshake needs is a full L2 writeback/invalidate per
// workgroup, which costs far more than the second launch.
//
// Output-major layout, y[N] = W[N x K] . x[K] (the *_nk entry points):
// each wave streams whole contiguous rows (gemv_rows_kernel, x read from the
// caches; gemv_rows_lds_kernel, x * gamma staged once per workgroup in LDS);
// no partial sums and a single launch.
#include "gemv_kernels.hpp"
#include "launch.hpp"

#include <algorithm>
#include <cstdlib>
#include <atomic>
#include <cstddef>
#include <memory>
#include <string>

namespace eng {
namespace {

using gemv::gemv_reduce_kernel;
using gemv::gemv_rows_kernel;
using gemv::gemv_rows_lds_kernel;
using gemv::gemv_rows_lds_multi_kernel;
using gemv::gemv_stream_kernel;

// K split of the reference-layout kernel for ncb column blocks: the grid is
// one round of resident workgroups (4 of the 512-thread workgroups per CU),
// every chunk a whole number of STEP-row loads and at least one unrolled step
// of all waves.
void kn_split(long long ncb, long long K, long long STEP, long long U, long long cus,
              long long& nsplit, long long& kchunk) {
  nsplit = 1;
  if (ncb < 2 * cus) {
    nsplit = (4 * cus) / ncb;
    nsplit = std::min(nsplit, (K + STEP * U - 1) / (STEP * U));
    nsplit = std::max(nsplit, 1LL);
  }
  kchunk = (K + nsplit - 1) / nsplit;
  kchunk = (kchunk + STEP - 1) / STEP * STEP;
  nsplit = (K + kchunk - 1) / kchunk;
}

// Reference-layout configuration: row segments of LPR lanes x 16 bytes; MX
// activation rows per launch (x row pitch K, y row pitch N).
template <typename WT, typename XT, typename YT, int VEC, int LPR, int WAVES, int U, bool RMS,
          int MX = 1>
void run_kn(const GemvArgs& a, hipStream_t stream) {
  constexpr int RPW = 64 / LPR;
  constexpr int STEP = WAVES * RPW;
  constexpr int CW = LPR * VEC;
  const long long N = a.N;
  const long long K = a.K;
  const long long ncb = (N + CW - 1) / CW;
  ENG_CHECK(ncb <= 0x7fffffffLL, "gemv: N too large for one launch");
  const long long cus = device_cu_count();

  // Split K so the grid is one round of resident workgroups (4 of these
  // 512-thread workgroups fit a CU: 2048 threads; their 44-58 VGPRs and 8 KiB
  // of LDS allow it), rounding down: a partly filled second round runs its
  // stragglers latency-bound (measured: 18-29% slower at 11008 x 4096 and
  // fp32 4096 x 4096). A chunk never has fewer rows than one unrolled step of
  // all waves.
  // The split does not depend on MX: a row's K chunks, and so its summation,
  // are the same in every batch, so each row of a small batch equals the
  // single-row result bit for bit. (Sizing the grid to the fewer resident
  // workgroups that 3 or 4 rows' accumulators allow measured 14% faster at
  // 4 x 11008 x 4096 -- 21.5 vs 24.6 us -- but would make results depend on
  // the batch.)
  long long nsplit = 0;
  long long kchunk = 0;
  kn_split(ncb, K, STEP, U, cus, nsplit, kchunk);
  ENG_CHECK(ncb * nsplit <= 0x7fffffffLL, "gemv: grid too large for one launch");

  const WT* W = static_cast<const WT*>(a.W);
  const XT* x = static_cast<const XT*>(a.x);
  YT* y = static_cast<YT*>(a.y);
  if (nsplit == 1) {
    gemv_stream_kernel<WT, XT, YT, VEC, LPR, WAVES, U, true, RMS, false, MX>
        <<<static_cast<unsigned>(ncb), WAVES * 64, 0, stream>>>(W, x, a.gamma, y, N, K, K, ncb,
                                                                 nullptr, nullptr, a.eps, nullptr);
    ENG_LAUNCH_CHECK();
    return;
  }
  // fp32 partial sums [nsplit x MX x N], then partial sums of squares [nsplit x MX].
  const std::size_t need = static_cast<std::size_t>(nsplit) * MX * (N + 1) * sizeof(float);
  float* partials = nullptr;
  std::unique_ptr<StreamScratch> ws;
  if (a.scratch != nullptr) {
    ENG_CHECK(need <= a.scratch_bytes,
              "gemv: the split-K partial sums need " + std::to_string(need) +
                  " bytes of scratch, more than the " + std::to_string(a.scratch_bytes) +
                  " bytes provided");
    partials = static_cast<float*>(a.scratch);
  } else {
    ws = std::make_unique<StreamScratch>(stream, need);
    partials = static_cast<float*>(ws->get());
  }
  float* partial_ss = partials + nsplit * MX * N;
  gemv_stream_kernel<WT, XT, YT, VEC, LPR, WAVES, U, true, RMS, true, MX>
      <<<static_cast<unsigned>(ncb * nsplit), WAVES * 64, 0, stream>>>(
          W, x, a.gamma, y, N, K, kchunk, ncb, partials, partial_ss, a.eps, nullptr);
  ENG_LAUNCH_CHECK();
  gemv_reduce_kernel<YT, RMS>
      <<<dim3(static_cast<unsigned>((N + 63) / 64), MX), gemv::kReduceWaves * 64, 0, stream>>>(
          partials, partial_ss, y, N, K, static_cast<int>(nsplit), a.eps, MX);
  ENG_LAUNCH_CHECK();
}

// 512-byte row segments (8 waves, 4 loads in flight per lane) for aligned
// vector rows; the scalar fallback (unaligned W or N not a multiple of the
// vector width) uses one lane per column.
template <typename WT, typename XT, typename YT, bool RMS, int MX = 1>
void dispatch_kn(const GemvArgs& a, hipStream_t stream) {
  constexpr int VMAX = 16 / static_cast<int>(sizeof(WT));
  const bool vec_ok = (a.N % VMAX == 0) && aligned_to(a.W, 16);
  if (vec_ok) {
    run_kn<WT, XT, YT, VMAX, 32, 8, 4, RMS, MX>(a, stream);
  } else {
    run_kn<WT, XT, YT, 1, 64, 4, 8, RMS, MX>(a, stream);
  }
}

// Scratch bytes run_kn takes for mx activation rows with the configuration
// dispatch_kn picks (0 when the K split is 1).
std::size_t kn_scratch_bytes_for(const GemvArgs& a, long long mx) {
  const long long wsize = a.w == Elem::F16 ? 2 : 4;
  const long long vmax = 16 / wsize;
  const bool vec_ok = (a.N % vmax == 0) && aligned_to(a.W, 16);
  const long long lpr = vec_ok ? 32 : 64;
  const long long vec = vec_ok ? vmax : 1;
  const long long waves = vec_ok ? 8 : 4;
  const long long u = vec_ok ? 4 : 8;
  const long long step = waves * (64 / lpr);
  const long long ncb = (a.N + lpr * vec - 1) / (lpr * vec);
  long long nsplit = 0;
  long long kchunk = 0;
  kn_split(ncb, a.K, step, u, device_cu_count(), nsplit, kchunk);
  if (nsplit == 1) return 0;
  return static_cast<std::size_t>(nsplit) * mx * (a.N + 1) * sizeof(float);
}

// Output-major register-kernel launches: 256-thread workgroups of 4 waves, R
// rows per wave.
template <typename WT, int VEC, int R, int U, bool RMS>
void launch_rows(const GemvArgs& a, hipStream_t stream) {
  const long long wgs = ((a.N + R - 1) / R + 3) / 4;
  ENG_CHECK(wgs <= 0x7fffffffLL, "gemv: N too large for one launch");
  gemv_rows_kernel<WT, VEC, R, U, RMS><<<static_cast<unsigned>(wgs), 256, 0, stream>>>(
      static_cast<const WT*>(a.W), static_cast<const float*>(a.x), a.gamma,
      static_cast<float*>(a.y), a.N, a.K, a.eps);
  ENG_LAUNCH_CHECK();
}

// LDS-staged output-major launches: workgroups of WAVES waves, R rows per
// wave, U loads per row in flight; NP > 0 selects the fixed-K form (K must be
// (NP - 1) * 512 + KT, groups of CH pieces).
template <typename WT, int R, int U, bool RMS, int WAVES, int NP = 0, int KT = 0, int CH = 0>
void launch_rows_lds(const GemvArgs& a, std::size_t lds_bytes, hipStream_t stream) {
  constexpr int VEC = 16 / static_cast<int>(sizeof(WT));
  if constexpr (NP > 0) {
    ENG_CHECK(a.K == (NP - 1) * 64LL * VEC + KT, "gemv: fixed-K kernel for another K");
  }
  const long long wgs = ((a.N + R - 1) / R + WAVES - 1) / WAVES;
  ENG_CHECK(wgs <= 0x7fffffffLL, "gemv: N too large for one launch");
  static std::atomic<bool> allowed[64] = {};
  allow_staged_lds(
      reinterpret_cast<const void*>(&gemv_rows_lds_kernel<WT, VEC, R, U, RMS, WAVES, NP, KT, CH>),
      allowed, lds_bytes);
  gemv_rows_lds_kernel<WT, VEC, R, U, RMS, WAVES, NP, KT, CH>
      <<<static_cast<unsigned>(wgs), WAVES * 64, lds_bytes, stream>>>(
          static_cast<const WT*>(a.W), static_cast<const float*>(a.x), a.gamma,
          static_cast<float*>(a.y), a.N, a.K, a.eps);
  ENG_LAUNCH_CHECK();
}

// Fixed-K fp16 rows past one resident round: gemv_rows_persist_kernel on
// two 16-wave workgroups per CU.
template <int NP, int KT, bool RMS>
void launch_rows_persist(const GemvArgs& a, hipStream_t stream) {
  ENG_CHECK(a.K == (NP - 1) * 512LL + KT, "gemv: fixed-K kernel for another K");
  const long long rows_wgs = (a.N + 15) / 16;
  const long long wgs = std::min<long long>(rows_wgs, 2LL * device_cu_count());
  const std::size_t lds = static_cast<std::size_t>(NP) * 512 * 4;
  static std::atomic<bool> allowed[64] = {};
  allow_staged_lds(reinterpret_cast<const void*>(&gemv::gemv_rows_persist_kernel<NP, KT, RMS>),
                   allowed, lds);
  gemv::gemv_rows_persist_kernel<NP, KT, RMS><<<static_cast<unsigned>(wgs), 1024, lds, stream>>>(
      static_cast<const _Float16*>(a.W), static_cast<const float*>(a.x), a.gamma,
      static_cast<float*>(a.y), a.N, a.eps);
  ENG_LAUNCH_CHECK();
}

// Fixed-K fp16 GEMV launches (no RMSNorm) of 16-wave workgroups with x
// staged by direct-to-LDS loads issued beside the first weight loads
// (gemv_rows_dma_kernel; the same bits as the register-staged
// gemv_rows_lds_kernel, which ENGINE_GEMV_NO_DMA=1 selects instead).
bool gemv_dma_enabled() {
  static const bool on = [] {
    const char* v = std::getenv("ENGINE_GEMV_NO_DMA");
    return !(v != nullptr && v[0] == '1');
  }();
  return on;
}

template <int NP, int KT, int CH, int WAVES>
void launch_rows_dma(const GemvArgs& a, hipStream_t stream) {
  ENG_CHECK(a.K == (NP - 1) * 512LL + KT, "gemv: fixed-K kernel for another K");
  const long long wgs = (a.N + WAVES - 1) / WAVES;
  ENG_CHECK(wgs <= 0x7fffffffLL, "gemv: N too large for one launch");
  const std::size_t lds = static_cast<std::size_t>(NP) * 512 * 4;
  static std::atomic<bool> allowed[64] = {};
  allow_staged_lds(reinterpret_cast<const void*>(&gemv::gemv_rows_dma_kernel<NP, KT, CH, WAVES>),
                   allowed, lds);
  gemv::gemv_rows_dma_kernel<NP, KT, CH, WAVES>
      <<<static_cast<unsigned>(wgs), 64 * WAVES, lds, stream>>>(
      static_cast<const _Float16*>(a.W), static_cast<const float*>(a.x),
      static_cast<float*>(a.y), a.N);
  ENG_LAUNCH_CHECK();
}

// Output-major configuration, from sweeps on MI355X at the decode shapes
// (cold weights): one wave per row fills the GPU once when N <= 16 x CUs
// (4 waves per SIMD), and 4 x 1 KiB loads per row in flight is then best;
// beyond that 8 in flight. For fp16 weights the x (and gamma) stream is
// larger than the weight row it meets, and once it no longer stays in the
// vector L1 (RMSNorm's x and gamma, or K > 4096) or rows outnumber resident
// waves, staging x * gamma in LDS wins: one row per wave, workgroups of 16
// waves (x staged once per 16 rows; 6-16% faster than 4-wave workgroups at
// 4096 x 4096 with RMSNorm, 11008 x 4096, 12288 x 4096 and 4096 x 11008),
// 4 loads per row in flight, 16 when K > 4096. x is staged for K up to 32768
// (128 KiB of LDS: at 8192 x 28672, 75 us against 95 us on the register
// kernel, whose x no longer stays in the caches). fp32 weights stay on the
// register kernel (2 rows per wave with RMSNorm), where the LDS variant
// measured slower.
template <typename WT, bool RMS>
void dispatch_nk(const GemvArgs& a, hipStream_t stream) {
  constexpr int VMAX = 16 / static_cast<int>(sizeof(WT));
  const bool vec_ok = (a.K % VMAX == 0) && aligned_to(a.W, 16) && aligned_to(a.x, 16) &&
                      (a.gamma == nullptr || aligned_to(a.gamma, 16));
  if (!vec_ok) {
    launch_rows<WT, 1, RMS ? 2 : 1, 8, RMS>(a, stream);
    return;
  }
  const long long one_round = 16LL * device_cu_count();
  if constexpr (sizeof(WT) == 2) {
    constexpr long long kPiece = 64 * VMAX;
    const long long padded = (a.K + kPiece - 1) / kPiece * kPiece;
    const bool fits = padded * 4 <= kStagedLdsMax;
    // Widths with a fixed-K form: the LDS-staged kernel once the rows give
    // every CU at least 8 waves (16-wave workgroups from 16 rows per CU, else
    // 8-wave) -- at 4096 x 4096 6.84 us against 7.31 us for the register
    // kernel, whose per-row re-read of x through the vector L1 costs 0.8 us.
    // Without RMSNorm, 16-wave workgroups stage x by direct-to-LDS loads that
    // overlap the first weight loads: 6.72 us against 6.92 at 4096 x 4096.
    // Rows longer than 4096 with at most one 16-wave workgroup per CU take
    // 8-wave workgroups (two per CU, the same waves): the down projection
    // 4096 x 11008 15.4 us against 16.0 (4096 x 4096 the same either way;
    // with RMSNorm, and for the fused gate / up, 8-wave workgroups measured
    // 6% slower). With RMSNorm x * gamma is staged from registers before the
    // weight stream starts: the early-start form (gemv_rows_rms_early_kernel,
    // which the fused gate / up uses) ran config 3 in 15.5 us on some boxes of
    // the pool and 17.5 us on others, against 15.8-15.9 us staged on both;
    // past one resident round the staged rows run on the persistent grid
    // (gemv_rows_persist_kernel, below).
    if (fits && (RMS || a.N >= one_round / 2 || a.K > 4096)) {
      const std::size_t lds = static_cast<std::size_t>(padded) * 4;
      const bool wide = RMS || a.N >= one_round || a.K > 4096;
      const bool fixed = with_fixed_k_f16(a.K, [&](auto fk) {
        using F = decltype(fk);
        if constexpr (RMS && F::NP <= 8) {
          // past one resident round: x * gamma staged once per resident
          // workgroup, each wave's next row streamed in behind its current one
          // (11008 x 4096: 15.3 us against 15.8-15.9 for a second round of
          // staged workgroups)
          if (a.N > 2 * one_round) {
            launch_rows_persist<F::NP, F::KT, RMS>(a, stream);
            return;
          }
        }
        if (!RMS && wide && gemv_dma_enabled()) {
          if (a.K > 4096 && a.N <= one_round) {
            // half a row's pieces in flight past 16 (4096 x 11008: 15.3 us
            // against 15.5 with all 22)
            launch_rows_dma<F::NP, F::KT, (F::CH1 > 16 ? F::CH1 / 2 : F::CH1), 8>(a, stream);
          } else {
            launch_rows_dma<F::NP, F::KT, F::CH1, 16>(a, stream);
          }
        } else if (wide) {
          launch_rows_lds<WT, 1, 4, RMS, 16, F::NP, F::KT, F::CH1>(a, lds, stream);
        } else {
          launch_rows_lds<WT, 1, 4, RMS, 8, F::NP, F::KT, F::CH1>(a, lds, stream);
        }
      });
      if (fixed) return;
    }
    if (fits && (RMS || a.N > one_round || a.K > 4096)) {
      const std::size_t lds = static_cast<std::size_t>(padded) * 4;
      if (a.K > 4096) {
        launch_rows_lds<WT, 1, 16, RMS, 16>(a, lds, stream);
      } else {
        launch_rows_lds<WT, 1, 4, RMS, 16>(a, lds, stream);
      }
      return;
    }
  }
  if constexpr (RMS) {
    launch_rows<WT, VMAX, 2, 8, true>(a, stream);
  } else if (sizeof(WT) == 2 && a.N <= one_round) {
    launch_rows<WT, VMAX, 1, 4, false>(a, stream);
  } else {
    launch_rows<WT, VMAX, 1, 8, false>(a, stream);
  }
}

}  // namespace

bool gemv_rms_early_enabled() {
  static const bool on = [] {
    const char* v = std::getenv("ENGINE_GEMV_NO_EARLY_RMS");
    return !(v != nullptr && v[0] == '1');
  }();
  return on;
}

// Per-device flags and counts shared by host threads: relaxed atomics (two
// threads may both set the attribute or read the count once; both are
// idempotent).
void allow_staged_lds(const void* kernel, std::atomic<bool> (&done)[64], std::size_t bytes) {
  if (bytes <= 64 * 1024) return;
  int dev = 0;
  ENG_HIP_CHECK(hipGetDevice(&dev));
  if (dev >= 0 && dev < 64 && done[dev].load(std::memory_order_relaxed)) return;
  ENG_HIP_CHECK(hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                    static_cast<int>(kStagedLdsMax)));
  if (dev >= 0 && dev < 64) done[dev].store(true, std::memory_order_relaxed);
}

int device_cu_count() {
  static std::atomic<int> cached[64] = {};
  int dev = 0;
  ENG_HIP_CHECK(hipGetDevice(&dev));
  if (dev >= 0 && dev < 64) {
    const int c = cached[dev].load(std::memory_order_relaxed);
    if (c > 0) return c;
  }
  int cus = 0;
  ENG_HIP_CHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
  if (cus <= 0) cus = 1;
  if (dev >= 0 && dev < 64) cached[dev].store(cus, std::memory_order_relaxed);
  return cus;
}

void launch_gemv(const GemvArgs& a, hipStream_t stream) {
  if (a.w_nk) {
    ENG_CHECK(a.x_elem == Elem::F32 && a.y_elem == Elem::F32, "gemv: unsupported element types");
    if (a.w == Elem::F16) {
      if (a.rms) {
        dispatch_nk<_Float16, true>(a, stream);
      } else {
        dispatch_nk<_Float16, false>(a, stream);
      }
    } else {
      if (a.rms) {
        dispatch_nk<float, true>(a, stream);
      } else {
        dispatch_nk<float, false>(a, stream);
      }
    }
    return;
  }
  if (a.w == Elem::F32) {
    ENG_CHECK(a.x_elem == Elem::F32 && a.y_elem == Elem::F32, "gemv: unsupported element types");
    if (a.rms) {
      dispatch_kn<float, float, float, true>(a, stream);
    } else {
      dispatch_kn<float, float, float, false>(a, stream);
    }
    return;
  }
  if (a.x_elem == Elem::F32 && a.y_elem == Elem::F32) {
    if (a.rms) {
      dispatch_kn<_Float16, float, float, true>(a, stream);
    } else {
      dispatch_kn<_Float16, float, float, false>(a, stream);
    }
    return;
  }
  ENG_CHECK(a.x_elem == Elem::F16 && a.y_elem == Elem::F16 && !a.rms,
            "gemv: unsupported element types");
  dispatch_kn<_Float16, _Float16, _Float16, false>(a, stream);
}

namespace {

// One round of resident workgroups, each looping over blocks of WAVES x R
// rows. fp16 weights: workgroups of 16 waves, one row per wave, one
// workgroup per CU when the staged rows take more than 32 KiB of LDS, else
// two (4 rows at 11008 x 4096: 20.6 us against 28.1 us for 4-wave
// workgroups, two per CU). fp32 weights: 4-wave workgroups, as many per CU as
// the LDS holds (up to 4).
template <typename WT, int R, int MX, bool RMS, int WAVES>
void launch_rows_multi(const GemvArgs& a, std::size_t lds_bytes, hipStream_t stream) {
  constexpr int VEC = 16 / static_cast<int>(sizeof(WT));
  const long long blocks = ((a.N + R - 1) / R + WAVES - 1) / WAVES;
  const long long per_cu =
      WAVES == 16 ? (lds_bytes <= 32 * 1024 ? 2 : 1)
                  : std::max<long long>(1, std::min<long long>(4, (160LL * 1024) / static_cast<long long>(lds_bytes + 64)));
  const long long wgs = std::min(blocks, per_cu * device_cu_count());
  static std::atomic<bool> allowed[64] = {};
  allow_staged_lds(
      reinterpret_cast<const void*>(&gemv_rows_lds_multi_kernel<WT, VEC, R, 4, MX, RMS, WAVES>),
      allowed, lds_bytes);
  gemv_rows_lds_multi_kernel<WT, VEC, R, 4, MX, RMS, WAVES>
      <<<static_cast<unsigned>(wgs), WAVES * 64, lds_bytes, stream>>>(
          static_cast<const WT*>(a.W), static_cast<const float*>(a.x), a.gamma,
          static_cast<float*>(a.y), a.N, a.K, a.eps);
  ENG_LAUNCH_CHECK();
}

template <typename WT, bool RMS>
void rows_multi(const GemvArgs& a, int mx, std::size_t lds, bool two, hipStream_t stream) {
  if constexpr (sizeof(WT) == 2) {
    switch (mx) {
      case 2: launch_rows_multi<WT, 1, 2, RMS, 16>(a, lds, stream); break;
      case 3: launch_rows_multi<WT, 1, 3, RMS, 16>(a, lds, stream); break;
      default: launch_rows_multi<WT, 1, 4, RMS, 16>(a, lds, stream); break;
    }
    return;
  }
  switch (mx * 2 + (two ? 1 : 0)) {
    case 4: launch_rows_multi<WT, 1, 2, RMS, 4>(a, lds, stream); break;
    case 5: launch_rows_multi<WT, 2, 2, RMS, 4>(a, lds, stream); break;
    case 6: launch_rows_multi<WT, 1, 3, RMS, 4>(a, lds, stream); break;
    case 7: launch_rows_multi<WT, 2, 3, RMS, 4>(a, lds, stream); break;
    case 8: launch_rows_multi<WT, 1, 4, RMS, 4>(a, lds, stream); break;
    default: launch_rows_multi<WT, 2, 4, RMS, 4>(a, lds, stream); break;
  }
}

}  // namespace

// Small-batch decode with output-major weights: y[M x N] = rows of x[M x K]
// times W[N x K]^T, in groups of up to kMultiRows rows that share one pass
// over W (gemv_rows_lds_multi_kernel; a group of one row is the single-row
// GEMV). The staged rows share an LDS budget of 128 KiB with fp16 weights (4
// rows at K = 4096, 2 at K = 11008) and 64 KiB with fp32 weights. Taken only
// when it needs at most kMaxPasses
// passes over W -- each pass costs about one GEMV, while the MFMA GEMM for a
// few rows costs about as much as that many passes (the GEMM pads M to its
// 64-row tile) -- and when the vector path's requirements hold; returns false
// otherwise and launches nothing.
bool launch_gemv_nk_rows(const GemvArgs& a, std::int64_t M, hipStream_t stream) {
  constexpr int kMultiRows = 4;
  constexpr long long kMaxPasses = 4;
  if (!a.w_nk || M < 1 || a.x_elem != Elem::F32 || a.y_elem != Elem::F32) return false;
  const long long kMaxLds = a.w == Elem::F16 ? kStagedLdsMax : 64 * 1024;
  const long long vmax = a.w == Elem::F16 ? 8 : 4;
  const bool vec_ok = (a.K % vmax == 0) && aligned_to(a.W, 16) && aligned_to(a.x, 16) &&
                      (a.gamma == nullptr || aligned_to(a.gamma, 16));
  if (!vec_ok) return false;
  const long long piece = 64 * vmax;
  const long long padded = (a.K + piece - 1) / piece * piece;
  const long long row_bytes = padded * 4;
  const long long fit = std::min<long long>(kMultiRows, kMaxLds / row_bytes);
  const long long per_pass = std::max<long long>(1, fit);
  const long long passes = (M + per_pass - 1) / per_pass;
  if (passes > kMaxPasses) return false;
  const bool two = a.N > 16LL * device_cu_count();
  for (long long m0 = 0; m0 < M; m0 += per_pass) {
    const int mx = static_cast<int>(std::min<long long>(per_pass, M - m0));
    GemvArgs g = a;
    g.x = static_cast<const float*>(a.x) + m0 * a.K;
    g.y = static_cast<float*>(a.y) + m0 * a.N;
    if (mx == 1) {
      launch_gemv(g, stream);
      continue;
    }
    const std::size_t lds = static_cast<std::size_t>(mx * row_bytes);
    if (a.w == Elem::F16) {
      if (a.rms) {
        rows_multi<_Float16, true>(g, mx, lds, two, stream);
      } else {
        rows_multi<_Float16, false>(g, mx, lds, two, stream);
      }
    } else {
      if (a.rms) {
        rows_multi<float, true>(g, mx, lds, two, stream);
      } else {
        rows_multi<float, false>(g, mx, lds, two, stream);
      }
    }
  }
  return true;
}

namespace {

template <typename WT, bool RMS>
void kn_rows(const GemvArgs& a, int mx, hipStream_t stream) {
  switch (mx) {
    case 2: dispatch_kn<WT, float, float, RMS, 2>(a, stream); break;
    case 3: dispatch_kn<WT, float, float, RMS, 3>(a, stream); break;
    default: dispatch_kn<WT, float, float, RMS, 4>(a, stream); break;
  }
}

}  // namespace

std::size_t gemv_kn_scratch_bytes(const GemvArgs& a, std::int64_t M) {
  return kn_scratch_bytes_for(a, std::min<std::int64_t>(M, 4));
}

// Small-batch decode with reference-layout weights A [K x N]: y[M x N] =
// x[M x K] . A, up to 4 rows per pass over A (the split-K kernel with MX
// activation rows; one row is the single-row GEMV). Same policy as
// launch_gemv_nk_rows: at most 4 passes, else false (the GEMM is left to run).
bool launch_gemv_kn_rows(const GemvArgs& a, std::int64_t M, hipStream_t stream) {
  constexpr long long kRows = 4;
  constexpr long long kMaxPasses = 4;
  if (a.w_nk || M < 1 || a.x_elem != Elem::F32 || a.y_elem != Elem::F32) return false;
  if ((M + kRows - 1) / kRows > kMaxPasses) return false;
  for (long long m0 = 0; m0 < M; m0 += kRows) {
    const int mx = static_cast<int>(std::min<long long>(kRows, M - m0));
    GemvArgs g = a;
    g.x = static_cast<const float*>(a.x) + m0 * a.K;
    g.y = static_cast<float*>(a.y) + m0 * a.N;
    if (mx == 1) {
      launch_gemv(g, stream);
    } else if (a.w == Elem::F16) {
      if (a.rms) {
        kn_rows<_Float16, true>(g, mx, stream);
      } else {
        kn_rows<_Float16, false>(g, mx, stream);
      }
    } else {
      if (a.rms) {
        kn_rows<float, true>(g, mx, stream);
      } else {
        kn_rows<float, false>(g, mx, stream);
      }
    }
  }
  return true;
}

namespace {

// act[MX x N] = SiLU(s xg . Wg) * (s xg . Wu) for MX rows, reference-layout
// Wg = a.W and Wu [K x N]: one stream launch over both matrices (DUAL, two
// column blocks per block of columns, with a single matrix's K split, so each
// plane's partial sums are those of the single-matrix kernel) and one reduce
// launch with the SwiGLU epilogue.
template <typename WT, int MX>
void run_kn_glu(const GemvArgs& a, const WT* Wu, hipStream_t stream) {
  constexpr int VEC = 16 / static_cast<int>(sizeof(WT));
  constexpr int LPR = 32;
  constexpr int WAVES = 8;
  constexpr int U = 4;
  constexpr int STEP = WAVES * (64 / LPR);
  constexpr int CW = LPR * VEC;
  const long long N = a.N;
  const long long K = a.K;
  const long long ncb = (N + CW - 1) / CW;
  long long nsplit = 0;
  long long kchunk = 0;
  kn_split(ncb, K, STEP, U, device_cu_count(), nsplit, kchunk);
  ENG_CHECK(2 * ncb * nsplit <= 0x7fffffffLL, "rmsnorm_linear_swiglu: grid too large for one launch");
  StreamScratch ws(stream, static_cast<std::size_t>(nsplit) * MX * (2 * N + 1) * sizeof(float));
  float* partials = static_cast<float*>(ws.get());
  float* partial_ss = partials + nsplit * MX * 2 * N;
  gemv_stream_kernel<WT, float, float, VEC, LPR, WAVES, U, true, true, true, MX, true>
      <<<static_cast<unsigned>(2 * ncb * nsplit), WAVES * 64, 0, stream>>>(
          static_cast<const WT*>(a.W), static_cast<const float*>(a.x), a.gamma, nullptr, N, K,
          kchunk, 2 * ncb, partials, partial_ss, a.eps, Wu);
  ENG_LAUNCH_CHECK();
  gemv_reduce_kernel<float, true, gemv::kReduceWaves, true>
      <<<dim3(static_cast<unsigned>((N + 63) / 64), MX), gemv::kReduceWaves * 64, 0, stream>>>(
          partials, partial_ss, static_cast<float*>(a.y), N, K, static_cast<int>(nsplit), a.eps, MX);
  ENG_LAUNCH_CHECK();
}

template <typename WT>
void kn_glu_rows(const GemvArgs& a, const void* Wu, int mx, hipStream_t stream) {
  const WT* u = static_cast<const WT*>(Wu);
  switch (mx) {
    case 1: run_kn_glu<WT, 1>(a, u, stream); break;
    case 2: run_kn_glu<WT, 2>(a, u, stream); break;
    case 3: run_kn_glu<WT, 3>(a, u, stream); break;
    default: run_kn_glu<WT, 4>(a, u, stream); break;
  }
}

}  // namespace

// Reference-layout FFN half for decode rows (a.rms, fp32 x and act, M rows
// of pitches K and N): passes of up to 4 rows, each one DUAL stream launch and
// one SwiGLU reduce (see run_kn_glu); every row equals its single-row result.
// Returns false, launching nothing, for more than 4 passes or unless both
// weight matrices take the vector path (N a multiple of the 16-byte vector,
// 16-byte aligned).
bool launch_gemv_kn_glu(const GemvArgs& a, const void* Wu, std::int64_t M, hipStream_t stream) {
  constexpr long long kRows = 4;
  constexpr long long kMaxPasses = 4;
  if (a.w_nk || !a.rms || M < 1 || a.x_elem != Elem::F32 || a.y_elem != Elem::F32) return false;
  if ((M + kRows - 1) / kRows > kMaxPasses) return false;
  const long long vmax = a.w == Elem::F16 ? 8 : 4;
  if (a.N % vmax != 0 || !aligned_to(a.W, 16) || !aligned_to(Wu, 16)) return false;
  for (long long m0 = 0; m0 < M; m0 += kRows) {
    const int mx = static_cast<int>(std::min<long long>(kRows, M - m0));
    GemvArgs g = a;
    g.x = static_cast<const float*>(a.x) + m0 * a.K;
    g.y = static_cast<float*>(a.y) + m0 * a.N;
    if (a.w == Elem::F16) {
      kn_glu_rows<_Float16>(g, Wu, mx, stream);
    } else {
      kn_glu_rows<float>(g, Wu, mx, stream);
    }
  }
  return true;
}

}  // namespace eng

using eng::guarded;

namespace {

// Shared body of the GEMV entry points: the reference's preconditions and
// messages (kernels/gemv.cu:116-128), then K == 0 zero-fill or the launch.
template <typename OutT>
void gemv_entry(const char* name, const void* A, const void* x, OutT* out, int64_t N, int64_t K,
                eng::Elem w, eng::Elem xe, eng::Elem ye, bool nk, eng_stream stream) {
  const std::string n(name);
  ENG_CHECK(A != nullptr, n + ": A is null");
  ENG_CHECK(x != nullptr, n + ": x is null");
  ENG_CHECK(out != nullptr, n + ": out is null");
  ENG_CHECK(N >= 0, n + ": N must be non-negative");
  ENG_CHECK(K >= 0, n + ": K must be non-negative");
  if (N == 0) return;
  hipStream_t s = eng::as_stream(stream);
  // An empty dot product is zero: K == 0 yields an all-zero output.
  if (K == 0) {
    eng::fill_zero_async(out, static_cast<std::size_t>(N) * sizeof(OutT), s);
    return;
  }
  eng::GemvArgs a;
  a.W = A;
  a.w = w;
  a.w_nk = nk;
  a.x = x;
  a.x_elem = xe;
  a.y = out;
  a.y_elem = ye;
  a.N = N;
  a.K = K;
  eng::launch_gemv(a, s);
}

}  // namespace

extern "C" {

int eng_gemv_f32(const float* A, const float* x, float* out, int64_t N, int64_t K,
                 eng_stream stream) {
  return guarded([&] {
    gemv_entry("gemv", A, x, out, N, K, eng::Elem::F32, eng::Elem::F32, eng::Elem::F32, false,
               stream);
  });
}

int eng_gemv_f16(const eng_half* A, const eng_half* x, eng_half* out, int64_t N, int64_t K,
                 eng_stream stream) {
  return guarded([&] {
    gemv_entry("gemv_fp16", A, x, out, N, K, eng::Elem::F16, eng::Elem::F16, eng::Elem::F16,
               false, stream);
  });
}

int eng_gemv_f16w(const eng_half* A, const float* x, float* out, int64_t N, int64_t K,
                  eng_stream stream) {
  return guarded([&] {
    gemv_entry("gemv_fp16", A, x, out, N, K, eng::Elem::F16, eng::Elem::F32, eng::Elem::F32,
               false, stream);
  });
}

int eng_gemv_f16w_nk(const eng_half* W, const float* x, float* y, int64_t N, int64_t K,
                     eng_stream stream) {
  return guarded([&] {
    gemv_entry("gemv_fp16", W, x, y, N, K, eng::Elem::F16, eng::Elem::F32, eng::Elem::F32, true,
               stream);
  });
}

int eng_gemv_f32_nk(const float* W, const float* x, float* y, int64_t N, int64_t K,
                    eng_stream stream) {
  return guarded([&] {
    gemv_entry("gemv", W, x, y, N, K, eng::Elem::F32, eng::Elem::F32, eng::Elem::F32, true,
               stream);
  });
}

}  // extern "C"
