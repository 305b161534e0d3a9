// ffn.hip -- fused RMSNorm + gate / up projections + SwiGLU, the first half of
// a Llama FFN:
//   act[r][n] = SiLU(xn[r] . Wg[:, n]) * (xn[r] . Wu[:, n]),  xn = RMSNorm(in) * gamma,
// with weights in the reference layout Wg, Wu [K x N] or output-major [N x K].
// The reference composes this from rmsnorm, two GEMVs / GEMMs and swiglu
// (tests/test_kernels.cu:2867-2898; its ADR 0006 defers fusing gate / up /
// SwiGLU on one weight stream).
//   * Output-major decode (M == 1, 16-byte aligned operands, K up to 32768
//     with fp16 weights, 16384 with fp32) runs gemv_rows_glu_kernel: one
//     launch that stages x * gamma in LDS,
//     streams each output's gate and up rows together and applies SiLU in the
//     epilogue, so gate and up never reach memory. A few rows (small-batch
//     decode) run gemv_rows_glu_multi_kernel: up to 4 rows per pass over Wg
//     and Wu, each row equal to its M = 1 result.
//   * Reference-layout decode (up to 16 rows, N a multiple of the 16-byte
//     vector, aligned weights) runs, per pass of up to 4 rows, the split-K
//     stream kernel over both matrices in one launch and the reduce with the
//     SwiGLU epilogue (launch_gemv_kn_glu): two launches where the composition
//     takes five, and the same bits.
//   * Otherwise gate and up are computed separately into the stream's scratch
//     arena -- single-row GEMVs, small-batch passes over W, or (more rows)
//     RMSNorm once and the MFMA GEMM: with fp16 weights (either layout) the
//     rows are split once into three fp16 planes and gate and up each run the
//     fp16-MFMA GEMM (launch_gemm_h3) -- and the SwiGLU kernel finishes.
// Preconditions and messages follow rmsnorm_linear; any zero dimension
// writes nothing.
#include "gemv_kernels.hpp"
#include "launch.hpp"

#include <algorithm>
#include <atomic>
#include <cstddef>

namespace eng {
namespace {

template <typename WT>
void rmsnorm_linear_swiglu(const float* in, const float* gamma, const WT* Wg, const WT* Wu,
                           float* act, int64_t M, int64_t N, int64_t K, float eps, Elem elem,
                           bool nk, eng_stream stream) {
  ENG_CHECK(M >= 0 && N >= 0 && K >= 0, "rmsnorm_linear_swiglu: negative dimension");
  ENG_CHECK(in != nullptr && Wg != nullptr && Wu != nullptr && act != nullptr,
            "rmsnorm_linear_swiglu: null device pointer");
  ENG_CHECK(eps >= 0.0f, "rmsnorm_linear_swiglu: eps must be non-negative");
  if (M == 0 || N == 0 || K == 0) return;
  hipStream_t s = as_stream(stream);

  constexpr int VEC = 16 / static_cast<int>(sizeof(WT));
  constexpr long long kPiece = 64 * VEC;
  constexpr long long kMaxLds = sizeof(WT) == 2 ? kStagedLdsMax : 64 * 1024;
  const long long padded = (K + kPiece - 1) / kPiece * kPiece;
  // Rows past the few-row kernels go to a GEMM. With fp16 Wg and Wu (either
  // layout, both aligned) that is the fp16-MFMA GEMM on the rows' three fp16
  // planes, split once for gate and up; else the rows normalised in fp32.
  // fp16 weights take it from kH3MinRows rows on.
  const bool h3 = elem == Elem::F16 && aligned_to(in, 16) &&
                  gemm_h3_applies(M, N, K, Wg, !nk) && gemm_h3_applies(M, N, K, Wu, !nk);
  // 5 to 64 rows (fp16 weights: 5 to 32): gate and up each in one pass over
  // its matrix on the matrix cores (skinny.hip), then SwiGLU.
  if (!h3 || M < kH3MinRows) {
    SkinnyArgs sk;
    sk.W = Wg;
    sk.w = elem;
    sk.w_nk = nk;
    sk.x = in;
    sk.gamma = gamma;
    sk.M = M;
    sk.N = N;
    sk.K = K;
    sk.rms = true;
    sk.eps = eps;
    SkinnyArgs sku = sk;
    sku.W = Wu;
    if (skinny_applies(sk) && skinny_applies(sku)) {
      const std::size_t mn = static_cast<std::size_t>(M) * static_cast<std::size_t>(N);
      // Level 1: the few-row launches lease their partial sums at level 0.
      StreamScratch gu(s, 2 * mn * sizeof(float), 1);
      float* gate = static_cast<float*>(gu.get());
      float* up = gate + mn;
      sk.y = gate;
      sku.y = up;
      launch_skinny(sk, s);
      launch_skinny(sku, s);
      launch_swiglu_f32(gate, up, act, static_cast<long long>(mn), s);
      return;
    }
  }
  if (!nk) {
    // Reference layout, up to 16 rows: per pass of up to 4 rows, one stream
    // launch over Wg and Wu and the reduce with the SwiGLU epilogue.
    GemvArgs gv;
    gv.W = Wg;
    gv.w = elem;
    gv.x = in;
    gv.gamma = gamma;
    gv.y = act;
    gv.N = N;
    gv.K = K;
    gv.rms = true;
    gv.eps = eps;
    if (launch_gemv_kn_glu(gv, Wu, M, s)) return;
  }
  const bool fused = nk && M == 1 && K % VEC == 0 && padded * 4 <= kMaxLds && aligned_to(Wg, 16) &&
                     aligned_to(Wu, 16) && aligned_to(in, 16) &&
                     (gamma == nullptr || aligned_to(gamma, 16));
  if (fused) {
    // One output (its gate and up rows) per wave; fp16 weights in workgroups of
    // 16 waves (x staged once per 16 outputs).
    constexpr int WAVES = sizeof(WT) == 2 ? 16 : 4;
    const long long wgs = (N + WAVES - 1) / WAVES;
    ENG_CHECK(wgs <= 0x7fffffffLL, "rmsnorm_linear_swiglu: N too large for one launch");
    const std::size_t lds = static_cast<std::size_t>(padded) * 4;
    if constexpr (sizeof(WT) == 2) {
      // fixed-K form for common widths (unmasked loads, 2 x CH2 in flight)
      const bool fixed = with_fixed_k_f16(K, [&](auto fk) {
        using F = decltype(fk);
        if (gemv_rms_early_enabled()) {
          // weight stream started before x * gamma is staged, the same bits;
          // 4 pieces per row in flight (11008 x 4096: 28.0 us against 29.1
          // staged first; rings of 2, 3, 5, 6 pieces 30.0, 28.2, 29.2, 30.7)
          auto kern = gemv::gemv_rows_rms_early_kernel<F::NP, F::KT, (F::NP < 4 ? F::NP : 4), true>;
          static std::atomic<bool> allowed_early[64] = {};
          const std::size_t lds_early = static_cast<std::size_t>(gemv::rms_early_lds_floats(F::NP)) * 4;
          allow_staged_lds(reinterpret_cast<const void*>(kern), allowed_early, lds_early);
          kern<<<static_cast<unsigned>(wgs), WAVES * 64, lds_early, s>>>(Wg, Wu, in, gamma, act, N, eps);
          ENG_LAUNCH_CHECK();
          return;
        }
        auto kern = gemv::gemv_rows_glu_kernel<WT, VEC, 1, 4, true, WAVES, F::NP, F::KT, F::CH2>;
        static std::atomic<bool> allowed_fixed[64] = {};
        allow_staged_lds(reinterpret_cast<const void*>(kern), allowed_fixed, lds);
        kern<<<static_cast<unsigned>(wgs), WAVES * 64, lds, s>>>(Wg, Wu, in, gamma, act, N, K, eps);
        ENG_LAUNCH_CHECK();
      });
      if (fixed) return;
    }
    static std::atomic<bool> allowed[64] = {};
    allow_staged_lds(reinterpret_cast<const void*>(&gemv::gemv_rows_glu_kernel<WT, VEC, 1, 4, true, WAVES>),
                     allowed, static_cast<std::size_t>(padded) * 4);
    gemv::gemv_rows_glu_kernel<WT, VEC, 1, 4, true, WAVES>
        <<<static_cast<unsigned>(wgs), WAVES * 64, static_cast<std::size_t>(padded) * 4, s>>>(
            Wg, Wu, in, gamma, act, N, K, eps);
    ENG_LAUNCH_CHECK();
    return;
  }
  // Small batch: up to 4 rows per pass over Wg and Wu, at most 4 passes.
  const long long fit = std::min<long long>(4, (64 * 1024) / (padded * 4));  // 64 KiB of staged rows
  const bool multi = nk && M > 1 && fit >= 2 && (M + fit - 1) / fit <= 4 && K % VEC == 0 &&
                     aligned_to(Wg, 16) && aligned_to(Wu, 16) && aligned_to(in, 16) &&
                     (gamma == nullptr || aligned_to(gamma, 16));
  if (multi) {
    // fp16 weights: workgroups of 16 waves, one per CU (4 rows at 11008 x
    // 4096: 36.4 us against 37.8 us for 4-wave workgroups, two per CU); fp32
    // weights: 4-wave workgroups, as many per CU as the LDS holds.
    constexpr int WAVES = sizeof(WT) == 2 ? 16 : 4;
    const long long blocks = (N + WAVES - 1) / WAVES;
    for (long long m0 = 0; m0 < M; m0 += fit) {
      const int mx = static_cast<int>(std::min<long long>(fit, M - m0));
      const float* xm = in + m0 * K;
      float* am = act + m0 * N;
      const std::size_t lds = static_cast<std::size_t>(mx * padded * 4);
      const long long per_cu =
          WAVES == 16 ? 1
                      : std::max<long long>(1, std::min<long long>(4, (160LL * 1024) / static_cast<long long>(lds + 64)));
      const unsigned grid = static_cast<unsigned>(std::min(blocks, per_cu * device_cu_count()));
      switch (mx) {
        case 1:
          gemv::gemv_rows_glu_kernel<WT, VEC, 1, 4, true, WAVES>
              <<<static_cast<unsigned>(blocks), WAVES * 64, lds, s>>>(Wg, Wu, xm, gamma, am, N, K, eps);
          break;
        case 2:
          gemv::gemv_rows_glu_multi_kernel<WT, VEC, 4, 2, true, WAVES>
              <<<grid, WAVES * 64, lds, s>>>(Wg, Wu, xm, gamma, am, N, K, eps);
          break;
        case 3:
          gemv::gemv_rows_glu_multi_kernel<WT, VEC, 4, 3, true, WAVES>
              <<<grid, WAVES * 64, lds, s>>>(Wg, Wu, xm, gamma, am, N, K, eps);
          break;
        default:
          gemv::gemv_rows_glu_multi_kernel<WT, VEC, 4, 4, true, WAVES>
              <<<grid, WAVES * 64, lds, s>>>(Wg, Wu, xm, gamma, am, N, K, eps);
          break;
      }
      ENG_LAUNCH_CHECK();
    }
    return;
  }

  const std::size_t mn = static_cast<std::size_t>(M) * static_cast<std::size_t>(N);
  const std::size_t mk = M > 1 ? static_cast<std::size_t>(M) * static_cast<std::size_t>(K) : 0;
  // The leading region holds the normalised rows (4 mk bytes) or the planes
  // and row scales (6 mk + 4 M bytes); gate and up follow, 256-byte aligned.
  const std::size_t plane_bytes = 3 * mk * sizeof(_Float16);
  const std::size_t lead =
      M > 1 ? (std::max(mk * sizeof(float), plane_bytes + static_cast<std::size_t>(M) * sizeof(float)) +
               255) & ~static_cast<std::size_t>(255)
            : 0;
  // Level 1: the GEMV launches below may lease split-K partials (level 0).
  StreamScratch scratch(s, lead + 2 * mn * sizeof(float), 1);
  char* base = static_cast<char*>(scratch.get());
  float* xn = reinterpret_cast<float*>(base);  // first: the GEMMs want it 16-byte aligned
  _Float16* planes = reinterpret_cast<_Float16*>(base);
  float* rscale = reinterpret_cast<float*>(base + plane_bytes);
  float* gate = reinterpret_cast<float*>(base + lead);
  float* up = gate + mn;
  bool normed = false;
  for (int half = 0; half < 2; ++half) {
    const void* W = half == 0 ? static_cast<const void*>(Wg) : static_cast<const void*>(Wu);
    float* out = half == 0 ? gate : up;
    GemvArgs gv;
    gv.W = W;
    gv.w = elem;
    gv.w_nk = nk;
    gv.x = in;
    gv.gamma = gamma;
    gv.y = out;
    gv.N = N;
    gv.K = K;
    gv.rms = true;
    gv.eps = eps;
    if (M == 1) {
      launch_gemv(gv, s);
    } else if (!(nk ? launch_gemv_nk_rows(gv, M, s) : launch_gemv_kn_rows(gv, M, s))) {
      // more than a few rows: normalise once, then the MFMA GEMM
      if (h3) {
        if (!normed) {
          launch_rmsnorm_split3(in, gamma, planes, rscale, M, K, eps, s);
          normed = true;
        }
        GemmH3Args h;
        h.P = planes;
        h.rscale = rscale;
        h.B = static_cast<const _Float16*>(W);
        h.C = out;
        h.M = M;
        h.N = N;
        h.K = K;
        h.b_kn = !nk;
        launch_gemm_h3(h, s);
        continue;
      }
      if (!normed) {
        launch_rmsnorm(in, gamma, xn, M, K, eps, s);
        normed = true;
      }
      GemmArgs g;
      g.A = xn;
      g.B = W;
      g.b = elem;
      g.b_nk = nk;
      g.C = out;
      g.M = M;
      g.N = N;
      g.K = K;
      launch_gemm(g, s);
    }
  }
  launch_swiglu_f32(gate, up, act, static_cast<long long>(mn), s);
}

}  // namespace
}  // namespace eng

extern "C" {

int eng_rmsnorm_linear_swiglu_f16w_nk(const float* in, const float* rms_weight,
                                      const eng_half* W_gate, const eng_half* W_up, float* act,
                                      int64_t M, int64_t N, int64_t K, float eps,
                                      eng_stream stream) {
  return eng::guarded([&] {
    eng::rmsnorm_linear_swiglu(in, rms_weight, reinterpret_cast<const _Float16*>(W_gate),
                               reinterpret_cast<const _Float16*>(W_up), act, M, N, K, eps,
                               eng::Elem::F16, true, stream);
  });
}

int eng_rmsnorm_linear_swiglu_f32_nk(const float* in, const float* rms_weight,
                                     const float* W_gate, const float* W_up, float* act,
                                     int64_t M, int64_t N, int64_t K, float eps,
                                     eng_stream stream) {
  return eng::guarded([&] {
    eng::rmsnorm_linear_swiglu(in, rms_weight, W_gate, W_up, act, M, N, K, eps, eng::Elem::F32,
                               true, stream);
  });
}

int eng_rmsnorm_linear_swiglu_f16w(const float* in, const float* rms_weight,
                                   const eng_half* W_gate, const eng_half* W_up, float* act,
                                   int64_t M, int64_t N, int64_t K, float eps,
                                   eng_stream stream) {
  return eng::guarded([&] {
    eng::rmsnorm_linear_swiglu(in, rms_weight, reinterpret_cast<const _Float16*>(W_gate),
                               reinterpret_cast<const _Float16*>(W_up), act, M, N, K, eps,
                               eng::Elem::F16, false, stream);
  });
}

int eng_rmsnorm_linear_swiglu_f32(const float* in, const float* rms_weight,
                                  const float* W_gate, const float* W_up, float* act, int64_t M,
                                  int64_t N, int64_t K, float eps, eng_stream stream) {
  return eng::guarded([&] {
    eng::rmsnorm_linear_swiglu(in, rms_weight, W_gate, W_up, act, M, N, K, eps, eng::Elem::F32,
                               false, stream);
  });
}

}  // extern "C"
