// rmsnorm_linear.hip -- fused RMSNorm + linear (reference kernels/rmsnorm_linear.cu:143-201).
//
//   out[r][n] = sum_k (in[r][k] * s_r * w_k) * W[k][n],  s_r = 1/sqrt(mean_k in[r][k]^2 + eps)
//
// The reference dispatches rmsnorm into pooled scratch and then gemv (M == 1)
// or the register-tiled GEMM (M > 1). Here M == 1 is one fused launch that
// never materialises the normalised row (the GEMV kernels with the sum of
// squares reduced alongside the dot products); M > 1 keeps the reference's
// structure -- rmsnorm into scratch, then the MFMA GEMM -- because the
// normalisation pass is a few microseconds of HBM traffic while applying gamma
// inside the GEMM repeats the multiply for every N-tile. The scratch is the
// stream's arena rather than the reference's pooled buffer (stream-ordered
// reuse without an event per call, and capturable in a HIP graph).
// Preconditions, messages and the "any zero dimension is a no-op" rule are
// the reference's. The *_nk entries take W output-major [N x K]
// (out = RMSNorm(in) . W^T), the layout the decode path streams best.
#include "launch.hpp"

#include <cstddef>

namespace eng {
namespace {

void rmsnorm_linear_any(const float* in, const float* rms_weight, const void* W, Elem w_elem,
                        bool nk, float* out, int64_t M, int64_t N, int64_t K, float eps,
                        eng_stream stream) {
  ENG_CHECK(M >= 0 && N >= 0 && K >= 0, "rmsnorm_linear: negative dimension");
  ENG_CHECK(in != nullptr && W != nullptr && out != nullptr,
            "rmsnorm_linear: null device pointer");
  ENG_CHECK(eps >= 0.0f, "rmsnorm_linear: eps must be non-negative");
  if (M == 0 || N == 0 || K == 0) return;
  hipStream_t s = as_stream(stream);
  GemvArgs g1;
  g1.W = W;
  g1.w = w_elem;
  g1.w_nk = nk;
  g1.x = in;
  g1.gamma = rms_weight;
  g1.y = out;
  g1.N = N;
  g1.K = K;
  g1.rms = true;
  g1.eps = eps;
  if (M == 1) {
    launch_gemv(g1, s);
    return;
  }
  // A few rows (small-batch decode): the rows share passes over W.
  if (nk ? launch_gemv_nk_rows(g1, M, s) : launch_gemv_kn_rows(g1, M, s)) return;
  StreamScratch normed(s, static_cast<std::size_t>(M) * static_cast<std::size_t>(K) * sizeof(float));
  float* xn = static_cast<float*>(normed.get());
  launch_rmsnorm(in, rms_weight, xn, M, K, eps, s);
  GemmArgs g;
  g.A = xn;
  g.B = W;
  g.b = w_elem;
  g.b_nk = nk;
  g.C = out;
  g.M = M;
  g.N = N;
  g.K = K;
  launch_gemm(g, s);
}

}  // namespace
}  // namespace eng

extern "C" {

int eng_rmsnorm_linear_f32(const float* in, const float* rms_weight, const float* W, float* out,
                           int64_t M, int64_t N, int64_t K, float eps, eng_stream stream) {
  return eng::guarded([&] {
    eng::rmsnorm_linear_any(in, rms_weight, W, eng::Elem::F32, false, out, M, N, K, eps, stream);
  });
}

int eng_rmsnorm_linear_f16w(const float* in, const float* rms_weight, const eng_half* W,
                            float* out, int64_t M, int64_t N, int64_t K, float eps,
                            eng_stream stream) {
  return eng::guarded([&] {
    eng::rmsnorm_linear_any(in, rms_weight, W, eng::Elem::F16, false, out, M, N, K, eps, stream);
  });
}

int eng_rmsnorm_linear_fused_direct_f32(const float* in, const float* rms_weight,
                                        const float* W, float* out, int64_t M, int64_t N,
                                        int64_t K, float eps, eng_stream stream) {
  return eng::guarded([&] {
    eng::rmsnorm_linear_any(in, rms_weight, W, eng::Elem::F32, false, out, M, N, K, eps, stream);
  });
}

int eng_rmsnorm_linear_f16w_nk(const float* in, const float* rms_weight, const eng_half* W,
                               float* out, int64_t M, int64_t N, int64_t K, float eps,
                               eng_stream stream) {
  return eng::guarded([&] {
    eng::rmsnorm_linear_any(in, rms_weight, W, eng::Elem::F16, true, out, M, N, K, eps, stream);
  });
}

int eng_rmsnorm_linear_f32_nk(const float* in, const float* rms_weight, const float* W,
                              float* out, int64_t M, int64_t N, int64_t K, float eps,
                              eng_stream stream) {
  return eng::guarded([&] {
    eng::rmsnorm_linear_any(in, rms_weight, W, eng::Elem::F32, true, out, M, N, K, eps, stream);
  });
}

}  // extern "C"
