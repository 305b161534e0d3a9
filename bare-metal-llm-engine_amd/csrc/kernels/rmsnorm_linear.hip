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
#include <mutex>
#include <string>

namespace eng {
namespace {

// Scratch of eng_rmsnorm_linear_f16w_noalloc: the split-K partial sums.
// Up to 4 rows (split-K GEMV passes): [nsplit][4][N] plus [nsplit][4] sums of
// squares, nsplit * N <= 4 x CUs x 256 (one round of 4 workgroups per CU, 256
// fp16 columns each): 4 MiB on a 256-CU MI355X. 5 to 16 rows (the few-row
// MFMA kernel): [nsplit][M][N] plus [nsplit][M], nsplit * N <= 2 x CUs x 128
// + 128 x ceil(N / 128) <= 4 x CUs x 128: 8 MiB at 16 rows on 256 CUs. Plus
// 64 KiB for the sums of squares and the split rounding. Each device holds
// its own copy for the life of the process.
constexpr std::size_t kNoAllocScratchBytes = (std::size_t{8} << 20) + (std::size_t{64} << 10);
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

// Device address of `scratch` on the current device, looked up once per
// device (the host-side name is a stand-in, never a device address).
void* noalloc_scratch_ptr() {
  constexpr int kMaxDevices = 64;
  static std::mutex mu;
  static void* ptrs[kMaxDevices] = {nullptr};
  int dev = 0;
  ENG_HIP_CHECK(hipGetDevice(&dev));
  ENG_CHECK(dev >= 0 && dev < kMaxDevices, "rmsnorm_linear_f16w_noalloc: device index out of range");
  std::lock_guard<std::mutex> lock(mu);
  if (ptrs[dev] == nullptr) {
    void* p = nullptr;
    ENG_HIP_CHECK(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    ENG_CHECK(p != nullptr, "rmsnorm_linear_f16w_noalloc: no device address for the scratch");
    ptrs[dev] = p;
  }
  return ptrs[dev];
}

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
  // fp16 W (either layout): the rows normalised into three fp16 planes, then
  // the fp16-MFMA GEMM (the same arithmetic as the FP32 GEMM on converted
  // weights, 16x the matrix rate per instruction); from kH3MinRows rows, or
  // below that for calls the few-row kernel and the row passes do not take.
  const bool h3 = w_elem == Elem::F16 && aligned_to(in, 16) && gemm_h3_applies(M, N, K, W, !nk);
  if (!h3 || M < kH3MinRows) {
    // 5 to 64 rows (fp16 W: 5 to 32): one pass over W on the matrix cores.
    SkinnyArgs sk = skinny_args(g1, M);
    if (skinny_applies(sk)) {
      launch_skinny(sk, s);
      return;
    }
    // 2 to 4 rows (small-batch decode, each row equal to its single-row call),
    // or rows the few-row kernel does not take: the rows share passes over W.
    if (nk ? launch_gemv_nk_rows(g1, M, s) : launch_gemv_kn_rows(g1, M, s)) return;
  }
  if (h3) {
    const std::size_t plane_bytes = 3 * static_cast<std::size_t>(M) * static_cast<std::size_t>(K) * 2;
    StreamScratch ws(s, plane_bytes + static_cast<std::size_t>(M) * sizeof(float));
    GemmH3Args h;
    h.P = static_cast<const _Float16*>(ws.get());
    h.rscale = reinterpret_cast<const float*>(static_cast<const char*>(ws.get()) + plane_bytes);
    h.B = static_cast<const _Float16*>(W);
    h.C = out;
    h.M = M;
    h.N = N;
    h.K = K;
    h.b_kn = !nk;
    launch_rmsnorm_split3(in, rms_weight, static_cast<_Float16*>(ws.get()),
                          const_cast<float*>(h.rscale), M, K, eps, s);
    launch_gemm_h3(h, s);
    return;
  }
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

// rmsnorm_linear_any for reference-layout fp16 W and M <= 16 rows, with the
// split-K partial sums (GEMV passes for up to 4 rows, the few-row MFMA kernel
// from 5) in the static `scratch` instead of the stream's arena:
// no allocation of any kind. The kernels and their configuration are
// eng_rmsnorm_linear_f16w's, so the results are the same bits.
void rmsnorm_linear_f16w_noalloc(const float* in, const float* rms_weight, const void* W,
                                 float* out, int64_t M, int64_t N, int64_t K, float eps,
                                 eng_stream stream) {
  ENG_CHECK(M >= 0 && N >= 0 && K >= 0, "rmsnorm_linear: negative dimension");
  ENG_CHECK(in != nullptr && W != nullptr && out != nullptr,
            "rmsnorm_linear: null device pointer");
  ENG_CHECK(eps >= 0.0f, "rmsnorm_linear: eps must be non-negative");
  ENG_CHECK(M <= 16, "rmsnorm_linear_f16w_noalloc: at most 16 rows (M = " + std::to_string(M) +
                         "); larger batches need eng_rmsnorm_linear_f16w");
  if (M == 0 || N == 0 || K == 0) return;
  GemvArgs g1;
  g1.W = W;
  g1.w = Elem::F16;
  g1.w_nk = false;
  g1.x = in;
  g1.gamma = rms_weight;
  g1.y = out;
  g1.N = N;
  g1.K = K;
  g1.rms = true;
  g1.eps = eps;
  hipStream_t s = as_stream(stream);
  SkinnyArgs sk = skinny_args(g1, M);
  const bool few_rows = M > 1 && skinny_applies(sk);
  const std::size_t need = few_rows ? skinny_scratch_bytes(sk) : gemv_kn_scratch_bytes(g1, M);
  ENG_CHECK(need <= kNoAllocScratchBytes,
            "rmsnorm_linear_f16w_noalloc: this shape needs " + std::to_string(need) +
                " bytes of scratch, more than the static " +
                std::to_string(kNoAllocScratchBytes) + " bytes");
  void* scratch_ptr = noalloc_scratch_ptr();
  if (few_rows) {
    sk.scratch = scratch_ptr;
    sk.scratch_bytes = kNoAllocScratchBytes;
    launch_skinny(sk, s);
    return;
  }
  g1.scratch = scratch_ptr;
  g1.scratch_bytes = kNoAllocScratchBytes;
  if (M == 1) {
    launch_gemv(g1, s);
    return;
  }
  const bool launched = launch_gemv_kn_rows(g1, M, s);
  ENG_CHECK(launched, "rmsnorm_linear_f16w_noalloc: internal error (small-batch path refused)");
}

}  // namespace
}  // namespace eng

extern "C" {

int eng_rmsnorm_linear_f16w_noalloc(const float* in, const float* rms_weight, const eng_half* W,
                                    float* out, int64_t M, int64_t N, int64_t K, float eps,
                                    eng_stream stream) {
  return eng::guarded([&] {
    eng::rmsnorm_linear_f16w_noalloc(in, rms_weight, W, out, M, N, K, eps, stream);
  });
}

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
