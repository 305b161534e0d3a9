#pragma once
//===----------------------------------------------------------------------===//
// engine/kernels.hpp -- C++17 launch API of the matrix-multiply path.
//
// Restates the reference's raw-pointer launchers (include/engine/kernels.hpp:
// 34-121; ADR docs/adr/0003) for the functions on this path, with the same
// names, argument order, defaults and error behaviour:
//   * every pointer is a DEVICE pointer; dimensions are std::int64_t;
//   * the last argument is the stream (nullptr = legacy default stream);
//   * launches are asynchronous; precondition failures throw
//     engine::EngineError with the reference's message substrings
//     ("null", "non-negative", "negative", "eps") before anything is launched.
// Each launcher forwards to the C-ABI in engine_hip.h. `engine::cuda` names
// the same namespace, so call sites written against the reference compile
// unchanged.
//===----------------------------------------------------------------------===//

#include <engine/check.hpp>
#include <engine/half.hpp>

#include <hip/hip_runtime_api.h>

#include <cstdint>

namespace engine {
namespace hip {

using engine::half;

namespace detail {
inline const eng_half* bits(const half* p) { return reinterpret_cast<const eng_half*>(p); }
inline eng_half* bits(half* p) { return reinterpret_cast<eng_half*>(p); }
}  // namespace detail

/// Row-wise RMSNorm: out = in / sqrt(mean(in^2) + eps) * weight. `weight` may be nullptr.
/// (reference kernels.hpp:61-63)
inline void rmsnorm(const float* in, const float* weight, float* out, std::int64_t rows,
                    std::int64_t cols, float eps, hipStream_t stream = nullptr) {
  ENGINE_ABI_CHECK(eng_rmsnorm_f32(in, weight, out, rows, cols, eps, stream));
}

/// C[M x N] = A[M x K] * B[K x N], row-major, fp32 accumulate; runs on the
/// FP32 matrix cores (the name is kept from the reference, kernels.hpp:77-81).
inline void matmul_register_tiled(const float* A, const float* B, float* C, std::int64_t M,
                                  std::int64_t N, std::int64_t K, hipStream_t stream = nullptr) {
  ENGINE_ABI_CHECK(eng_matmul_f32(A, B, C, M, N, K, stream));
}

/// out[N] = x[K] * A[K x N], row-major (reference kernels.hpp:83-86).
inline void gemv(const float* A, const float* x, float* out, std::int64_t N, std::int64_t K,
                 hipStream_t stream = nullptr) {
  ENGINE_ABI_CHECK(eng_gemv_f32(A, x, out, N, K, stream));
}

/// out[M x N] = RMSNorm(in[M x K], rms_weight, eps) * W[K x N]; `rms_weight` may
/// be nullptr (reference kernels.hpp:92-99). One fused kernel for every M.
inline void rmsnorm_linear(const float* in, const float* rms_weight, const float* W, float* out,
                           std::int64_t M, std::int64_t N, std::int64_t K, float eps,
                           hipStream_t stream = nullptr) {
  ENGINE_ABI_CHECK(eng_rmsnorm_linear_f32(in, rms_weight, W, out, M, N, K, eps, stream));
}

/// fp16-weight overload (fp32 activations in and out).
inline void rmsnorm_linear(const float* in, const float* rms_weight, const half* W, float* out,
                           std::int64_t M, std::int64_t N, std::int64_t K, float eps,
                           hipStream_t stream = nullptr) {
  ENGINE_ABI_CHECK(
      eng_rmsnorm_linear_f16w(in, rms_weight, detail::bits(W), out, M, N, K, eps, stream));
}

/// The reference's benchmarking entry that forces its fused kernel
/// (kernels.hpp:101-104); every M is fused here, so it is rmsnorm_linear.
inline void rmsnorm_linear_fused_direct(const float* in, const float* rms_weight, const float* W,
                                        float* out, std::int64_t M, std::int64_t N,
                                        std::int64_t K, float eps, hipStream_t stream = nullptr) {
  ENGINE_ABI_CHECK(
      eng_rmsnorm_linear_fused_direct_f32(in, rms_weight, W, out, M, N, K, eps, stream));
}

/// out[N] = x[K] * A[K x N] in FP16 storage with fp32 accumulation; out rounded
/// to nearest even (reference kernels.hpp:118-121).
inline void gemv_fp16(const half* A, const half* x, half* out, std::int64_t N, std::int64_t K,
                      hipStream_t stream = nullptr) {
  ENGINE_ABI_CHECK(eng_gemv_f16(detail::bits(A), detail::bits(x), detail::bits(out), N, K, stream));
}

/// fp16-weight overload with fp32 activations in and out (decode with fp16 weights).
inline void gemv_fp16(const half* A, const float* x, float* out, std::int64_t N, std::int64_t K,
                      hipStream_t stream = nullptr) {
  ENGINE_ABI_CHECK(eng_gemv_f16w(detail::bits(A), x, out, N, K, stream));
}

/// Output-major weights (additive; no reference counterpart): y[N] = W[N x K] * x[K].
inline void gemv_nk(const half* W, const float* x, float* y, std::int64_t N, std::int64_t K,
                    hipStream_t stream = nullptr) {
  ENGINE_ABI_CHECK(eng_gemv_f16w_nk(detail::bits(W), x, y, N, K, stream));
}
inline void gemv_nk(const float* W, const float* x, float* y, std::int64_t N, std::int64_t K,
                    hipStream_t stream = nullptr) {
  ENGINE_ABI_CHECK(eng_gemv_f32_nk(W, x, y, N, K, stream));
}

/// Weight layout conversion (additive): dst[cols x rows] = src[rows x cols]^T,
/// bits unchanged. Converts a reference-layout A [K x N] once into the
/// output-major W [N x K] of gemv_nk / rmsnorm_linear_nk.
inline void transpose(const half* src, half* dst, std::int64_t rows, std::int64_t cols,
                      hipStream_t stream = nullptr) {
  ENGINE_ABI_CHECK(eng_transpose_f16(detail::bits(src), detail::bits(dst), rows, cols, stream));
}
inline void transpose(const float* src, float* dst, std::int64_t rows, std::int64_t cols,
                      hipStream_t stream = nullptr) {
  ENGINE_ABI_CHECK(eng_transpose_f32(src, dst, rows, cols, stream));
}

/// Output-major weights: out[M x N] = RMSNorm(in[M x K], rms_weight, eps) * W[N x K]^T.
inline void rmsnorm_linear_nk(const float* in, const float* rms_weight, const half* W, float* out,
                              std::int64_t M, std::int64_t N, std::int64_t K, float eps,
                              hipStream_t stream = nullptr) {
  ENGINE_ABI_CHECK(
      eng_rmsnorm_linear_f16w_nk(in, rms_weight, detail::bits(W), out, M, N, K, eps, stream));
}
inline void rmsnorm_linear_nk(const float* in, const float* rms_weight, const float* W, float* out,
                              std::int64_t M, std::int64_t N, std::int64_t K, float eps,
                              hipStream_t stream = nullptr) {
  ENGINE_ABI_CHECK(eng_rmsnorm_linear_f32_nk(in, rms_weight, W, out, M, N, K, eps, stream));
}

/// out[i] = a[i] + b[i], bit-exact (reference kernels.hpp:47-50).
inline void vector_add(const float* a, const float* b, float* out, std::int64_t n,
                       hipStream_t stream = nullptr) {
  ENGINE_ABI_CHECK(eng_vector_add_f32(a, b, out, n, stream));
}

/// sum_out = x + residual; norm_out = RMSNorm(sum_out, weight, eps); `weight`
/// may be nullptr (reference kernels.hpp:106-112).
inline void residual_rmsnorm(const float* x, const float* residual, const float* weight,
                             float* norm_out, float* sum_out, std::int64_t rows,
                             std::int64_t cols, float eps, hipStream_t stream = nullptr) {
  ENGINE_ABI_CHECK(
      eng_residual_rmsnorm_f32(x, residual, weight, norm_out, sum_out, rows, cols, eps, stream));
}

/// out[i] = SiLU(gate[i]) * up[i] (reference kernels.hpp:138-142).
inline void swiglu(const float* gate, const float* up, float* out, std::int64_t n,
                   hipStream_t stream = nullptr) {
  ENGINE_ABI_CHECK(eng_swiglu_f32(gate, up, out, n, stream));
}
inline void swiglu_fp16(const half* gate, const half* up, half* out, std::int64_t n,
                        hipStream_t stream = nullptr) {
  ENGINE_ABI_CHECK(
      eng_swiglu_f16(detail::bits(gate), detail::bits(up), detail::bits(out), n, stream));
}

/// Gate / up half of a SwiGLU FFN with output-major weights [N x K]:
/// act = SiLU(RMSNorm(in) * W_gate^T) * (RMSNorm(in) * W_up^T). One launch at
/// M == 1 (additive; the reference composes rmsnorm, two GEMVs and swiglu).
inline void rmsnorm_linear_swiglu_nk(const float* in, const float* rms_weight, const half* W_gate,
                                     const half* W_up, float* act, std::int64_t M, std::int64_t N,
                                     std::int64_t K, float eps, hipStream_t stream = nullptr) {
  ENGINE_ABI_CHECK(eng_rmsnorm_linear_swiglu_f16w_nk(in, rms_weight, detail::bits(W_gate),
                                                     detail::bits(W_up), act, M, N, K, eps,
                                                     stream));
}
inline void rmsnorm_linear_swiglu_nk(const float* in, const float* rms_weight, const float* W_gate,
                                     const float* W_up, float* act, std::int64_t M, std::int64_t N,
                                     std::int64_t K, float eps, hipStream_t stream = nullptr) {
  ENGINE_ABI_CHECK(
      eng_rmsnorm_linear_swiglu_f32_nk(in, rms_weight, W_gate, W_up, act, M, N, K, eps, stream));
}

/// The same with reference-layout weights [K x N] (rmsnorm_linear's layout):
/// two launches at M == 1 instead of the composition's five, same result.
inline void rmsnorm_linear_swiglu(const float* in, const float* rms_weight, const half* W_gate,
                                  const half* W_up, float* act, std::int64_t M, std::int64_t N,
                                  std::int64_t K, float eps, hipStream_t stream = nullptr) {
  ENGINE_ABI_CHECK(eng_rmsnorm_linear_swiglu_f16w(in, rms_weight, detail::bits(W_gate),
                                                  detail::bits(W_up), act, M, N, K, eps, stream));
}
inline void rmsnorm_linear_swiglu(const float* in, const float* rms_weight, const float* W_gate,
                                  const float* W_up, float* act, std::int64_t M, std::int64_t N,
                                  std::int64_t K, float eps, hipStream_t stream = nullptr) {
  ENGINE_ABI_CHECK(
      eng_rmsnorm_linear_swiglu_f32(in, rms_weight, W_gate, W_up, act, M, N, K, eps, stream));
}

namespace detail {

/// FlashDecoding with GQA K / V sharing switched explicitly (reference
/// kernels.hpp:169-174, for ablations).
inline void attention_decode_with_mode(const half* q, const half* k, const half* v, half* out,
                                       std::int64_t kv_len, std::int64_t n_heads,
                                       std::int64_t n_kv_heads, std::int64_t head_dim,
                                       std::int64_t kv_head_stride, float scale, int split_kv,
                                       bool share_gqa_kv, hipStream_t stream) {
  ENGINE_ABI_CHECK(eng_attention_decode_with_mode_f16(
      bits(q), bits(k), bits(v), bits(out), kv_len, n_heads, n_kv_heads, head_dim,
      kv_head_stride, scale, split_kv, share_gqa_kv ? 1 : 0, stream));
}

/// fp32 -> fp16 and back, elementwise (reference kernels.hpp:176-180).
inline void cast_f32_to_f16(const float* in, half* out, std::int64_t n,
                            hipStream_t stream = nullptr) {
  ENGINE_ABI_CHECK(eng_cast_f32_to_f16(in, bits(out), n, stream));
}
inline void cast_f16_to_f32(const half* in, float* out, std::int64_t n,
                            hipStream_t stream = nullptr) {
  ENGINE_ABI_CHECK(eng_cast_f16_to_f32(bits(in), out, n, stream));
}

/// Token-major K / V -> head-major KV caches (reference kernels.hpp:182-188).
inline void kv_cache_write(const half* k_new, const half* v_new, half* k_cache, half* v_cache,
                           std::int64_t s_new, std::int64_t n_kv_heads, std::int64_t head_dim,
                           std::int64_t pos_offset, std::int64_t kv_max_seq_len,
                           hipStream_t stream = nullptr) {
  ENGINE_ABI_CHECK(eng_kv_cache_write_f16(bits(k_new), bits(v_new), bits(k_cache), bits(v_cache),
                                          s_new, n_kv_heads, head_dim, pos_offset,
                                          kv_max_seq_len, stream));
}

}  // namespace detail

/// Single-token decode attention, split-KV FlashDecoding over an fp16 KV
/// cache; split_kv = 0 chooses the split count (reference kernels.hpp:190-194).
inline void attention_decode(const half* q, const half* k, const half* v, half* out,
                             std::int64_t kv_len, std::int64_t n_heads, std::int64_t n_kv_heads,
                             std::int64_t head_dim, std::int64_t kv_head_stride, float scale,
                             int split_kv = 0, hipStream_t stream = nullptr) {
  ENGINE_ABI_CHECK(eng_attention_decode_f16(detail::bits(q), detail::bits(k), detail::bits(v),
                                            detail::bits(out), kv_len, n_heads, n_kv_heads,
                                            head_dim, kv_head_stride, scale, split_kv, stream));
}

}  // namespace hip

// Call sites written against the reference use engine::cuda::...
namespace cuda = hip;

}  // namespace engine
