// launch.hpp -- internal launchers shared by the C-ABI entry points.
// Callers have validated pointers and dimensions and handled the zero-size
// cases; these only pick a kernel configuration and launch on `stream`.
#pragma once

#include "../engine_internal.hpp"

#include <atomic>
#include <cstddef>
#include <cstdint>

namespace eng {

enum class Elem { F32, F16 };

// out[N] = sum_k xs_k * W[k][n]  with  xs_k = x_k * gamma_k (gamma optional)
// (or sum_k W[n][k] xs_k when w_nk);
// with rms, out is further multiplied by 1/sqrt(sum_k x_k^2 / K + eps).
struct GemvArgs {
  const void* W = nullptr;
  Elem w = Elem::F32;
  bool w_nk = false;  // W stored output-major [N x K]: y = W . x
  const void* x = nullptr;
  Elem x_elem = Elem::F32;
  const float* gamma = nullptr;
  void* y = nullptr;
  Elem y_elem = Elem::F32;
  std::int64_t N = 0;
  std::int64_t K = 0;
  bool rms = false;
  float eps = 0.0f;
  // Caller-provided device scratch for the reference-layout split-K partial
  // sums (used instead of the stream's arena when set; a launch that needs
  // more than scratch_bytes fails with an error and launches nothing).
  void* scratch = nullptr;
  std::size_t scratch_bytes = 0;
};
void launch_gemv(const GemvArgs& a, hipStream_t stream);
// Largest dynamic LDS of the staged-activation kernels with fp16 weights:
// 128 KiB (x of up to K = 32768 for one row, two rows at K = 11008 for a
// small-batch pass; one 16-wave workgroup per CU past 64 KiB).
constexpr long long kStagedLdsMax = 128 * 1024;
// Widths K with a compile-time form of the fp16 LDS-staged decode kernels
// (dot_rows_lds_fixed): K = (NP - 1) * 512 + KT, streamed in groups of CH1
// pieces for one weight row per wave and CH2 for two (the FFN's gate and up).
// The groups keep a wave's loads in flight within the VGPRs of 16-wave
// workgroups (CH1 x 4 and 2 CH2 x 4 registers of weights).
template <int NP_, int KT_, int CH1_, int CH2_>
struct FixedK {
  static constexpr int NP = NP_;
  static constexpr int KT = KT_;
  static constexpr int CH1 = CH1_;
  static constexpr int CH2 = CH2_;
};
// Calls f(FixedK<...>{}) and returns true when K has a fixed form.
template <class F>
bool with_fixed_k_f16(long long K, F&& f) {
  switch (K) {
    case 2048: f(FixedK<4, 512, 4, 4>{}); return true;
    case 4096: f(FixedK<8, 512, 8, 8>{}); return true;
    case 5120: f(FixedK<10, 512, 10, 5>{}); return true;
    case 8192: f(FixedK<16, 512, 16, 8>{}); return true;
    case 11008: f(FixedK<22, 256, 22, 8>{}); return true;
    case 14336: f(FixedK<28, 512, 14, 7>{}); return true;
    default: return false;
  }
}
// False when ENGINE_GEMV_NO_EARLY_RMS=1: the fixed-K fp16 fused gate / up
// kernel then stages x * gamma before starting the weight stream (the same
// bits, for comparison).
bool gemv_rms_early_enabled();
// Past 64 KiB a kernel's dynamic LDS must be allowed explicitly: once per
// device per kernel (`done` is that kernel's flag array); a no-op below.
void allow_staged_lds(const void* kernel, std::atomic<bool> (&done)[64], std::size_t bytes);
// Output-major W only: y[M x N] = x[M x K] . W^T for a few rows (x and y
// row-major, pitches K and N; a.x / a.y point at row 0), in groups that share
// a pass over W. Returns false, launching nothing, when the shape is better
// left to the GEMM (or the vector path's alignment requirements fail).
bool launch_gemv_nk_rows(const GemvArgs& a, std::int64_t M, hipStream_t stream);
// Reference-layout W [K x N] counterpart of launch_gemv_nk_rows.
bool launch_gemv_kn_rows(const GemvArgs& a, std::int64_t M, hipStream_t stream);
// Largest scratch (bytes) that launch_gemv / launch_gemv_kn_rows take for the
// split-K partial sums of a reference-layout call over M rows (M <= 16; the
// first pass, of min(M, 4) rows, needs the most).
std::size_t gemv_kn_scratch_bytes(const GemvArgs& a, std::int64_t M);
// Reference-layout gate / up + SwiGLU for M decode rows: a.y = SiLU(RMSNorm(a.x)
// . a.W) * (RMSNorm(a.x) . Wu), equal bit for bit to the two RMSNorm + linear
// calls and swiglu. Returns false, launching nothing, for more than 16 rows or
// when the vector path's requirements fail.
bool launch_gemv_kn_glu(const GemvArgs& a, const void* Wu, std::int64_t M, hipStream_t stream);

// Few-row linear layers on FP32 MFMA (skinny.hip): y[M x N] = x'[M x K] . W
// (W [K x N]) or x' . W^T (w_nk, W [N x K]), x' = x (or, with rms, x * gamma
// with row m scaled by 1/sqrt(mean_k x[m][k]^2 + eps) after the sum), W read
// once for all rows. Rows of one call are independent of each other and of M.
constexpr std::int64_t kSkinnyMinRows = 5;
constexpr std::int64_t kSkinnyMaxRows = 64;     // fp32 weights
constexpr std::int64_t kSkinnyMaxRowsF16 = 32;  // fp16 weights
// fp16 weights from this many rows take the fp16-MFMA GEMM on three fp16
// planes (exact products, 64 x 128 tiles up to 64 rows) instead of the
// few-row kernel, which takes 16-row blocks (33-64 x 11008 x 4096: 41-50 us
// against 37.5-42 cold); the few-row kernel keeps fp16 weights at 5-32 rows
// and fp32 weights at 5-64.
constexpr std::int64_t kH3MinRows = kSkinnyMaxRowsF16 + 1;
struct SkinnyArgs {
  const void* W = nullptr;
  Elem w = Elem::F32;
  bool w_nk = false;
  const float* x = nullptr;
  const float* gamma = nullptr;  // rms only (optional)
  float* y = nullptr;
  std::int64_t M = 0;
  std::int64_t N = 0;
  std::int64_t K = 0;
  bool rms = false;
  float eps = 0.0f;
  // Caller-provided device scratch for the split-K partial sums (instead of
  // the stream's arena; a launch needing more than scratch_bytes fails).
  void* scratch = nullptr;
  std::size_t scratch_bytes = 0;
};
// Whether the few-row kernel takes this call: kSkinnyMinRows <= M <=
// kSkinnyMaxRows (fp16 W: kSkinnyMaxRowsF16), K % 8 == 0, N a multiple of the 16-byte vector in the
// reference layout, and 16-byte aligned W, x and gamma.
bool skinny_applies(const SkinnyArgs& a);
// Scratch bytes launch_skinny takes (0 when K is not split).
std::size_t skinny_scratch_bytes(const SkinnyArgs& a);
void launch_skinny(const SkinnyArgs& a, hipStream_t stream);
// The few-row form of an M-row GEMV-style call (fp32 x and y only; other
// element types give M = 0, which no kernel takes).
inline SkinnyArgs skinny_args(const GemvArgs& g, std::int64_t M) {
  SkinnyArgs a;
  a.W = g.W;
  a.w = g.w;
  a.w_nk = g.w_nk;
  a.x = static_cast<const float*>(g.x);
  a.gamma = g.rms ? g.gamma : nullptr;
  a.y = static_cast<float*>(g.y);
  a.M = (g.x_elem == Elem::F32 && g.y_elem == Elem::F32) ? M : 0;
  a.N = g.N;
  a.K = g.K;
  a.rms = g.rms;
  a.eps = g.eps;
  return a;
}

// C[M x N] = A'[M x K] . B[K x N] on FP32 MFMA, where A' = A with column k
// scaled by gamma_k when gamma is given; with rms, row r of C is further
// multiplied by 1/sqrt(sum_k A[r][k]^2 / K + eps).
struct GemmArgs {
  const float* A = nullptr;
  const void* B = nullptr;
  Elem b = Elem::F32;
  bool b_nk = false;  // B given as [N x K] (C = A . B^T)
  float* C = nullptr;
  std::int64_t M = 0;
  std::int64_t N = 0;
  std::int64_t K = 0;
};
void launch_gemm(const GemmArgs& a, hipStream_t stream);

// out[r][c] = in[r][c] * s_r * weight[c] (weight optional).
void launch_rmsnorm(const float* in, const float* weight, float* out, long long rows,
                    long long cols, float eps, hipStream_t stream);

// The same rows scaled by 2^e_r (largest |value| of each row in [2^14, 2^15))
// as three fp16 planes, p = 0..2, that sum to the scaled value; rscale[r] =
// 2^-e_r. Each plane is K-blocked, [cols / 32][rows][32]: value (r, c) at
// planes[p rows cols + ((c / 32) rows + r) 32 + c % 32]. Needs cols % 32 == 0
// and 16-byte aligned in and planes.
void launch_rmsnorm_split3(const float* in, const float* weight, _Float16* planes, float* rscale,
                           long long rows, long long cols, float eps, hipStream_t stream);

// C[M x N] = diag(rscale) (P[0] + P[1] + P[2]) . B^T on fp16 MFMA, B fp16
// [N x K] (output-major weights), or C = diag(rscale) (P[0] + P[1] + P[2]) . B
// with B fp16 [K x N] (the reference layout, b_kn); P the K-blocked planes of
// launch_rmsnorm_split3.
// Needs K % 32 == 0 and 16-byte aligned P and B; [K x N] B also N % 8 == 0
// and at most 2^31 - 1 bytes.
struct GemmH3Args {
  const _Float16* P = nullptr;
  const float* rscale = nullptr;
  const _Float16* B = nullptr;
  float* C = nullptr;
  std::int64_t M = 0;
  std::int64_t N = 0;
  std::int64_t K = 0;
  bool b_kn = false;
};
bool gemm_h3_applies(std::int64_t M, std::int64_t N, std::int64_t K, const void* B, bool b_kn);
void launch_gemm_h3(const GemmH3Args& a, hipStream_t stream);

// out[i] = SiLU(g[i]) * u[i] in fp32.
void launch_swiglu_f32(const float* g, const float* u, float* out, long long n,
                       hipStream_t stream);

// Number of compute units of the current device (cached per device).
int device_cu_count();

}  // namespace eng
