/*
 * oracle.h -- TEST INFRASTRUCTURE ONLY. CPU restatement of the reference's
 * scalar oracle for the matrix-multiply path (reference src/cpu_ref/ and
 * include/engine/cpu_ref.hpp). Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load it, and only as the checker or the
 * timed CPU baseline; the engine never calls it.
 *
 * Semantics (reference include/engine/cpu_ref.hpp:14-17): row-major,
 * contiguous; scalar loops with double accumulators; no threads, no SIMD
 * intrinsics; outputs rounded to float (or to half, round-to-nearest-even).
 *
 * Parity pinning of every function is listed in oracle.c's header.
 */
#ifndef ENGINE_ORACLE_H
#define ENGINE_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* C[M x N] = A[M x K] . B[K x N] (reference src/cpu_ref/matmul_cpu.cpp:16-29). */
void orc_matmul(const float* A, const float* B, float* C, int64_t M, int64_t N, int64_t K);

/* out[N] = x[K] . A[K x N] (reference src/cpu_ref/gemv_cpu.cpp:15-23). */
void orc_gemv(const float* A, const float* x, float* out, int64_t N, int64_t K);

/* Half A, x, out; double accumulate; out rounded to half
 * (reference src/cpu_ref/gemv_cpu.cpp:25-35). */
void orc_gemv_fp16(const uint16_t* A, const uint16_t* x, uint16_t* out, int64_t N, int64_t K);

/* Half A, fp32 x and out, double accumulate: the fp16-weight decode GEMV of
 * the benchmark configs, stated in the same form as orc_gemv_fp16. */
void orc_gemv_f16w(const uint16_t* A, const float* x, float* out, int64_t N, int64_t K);

/* out = in / sqrt(mean(in^2) + eps) * weight (weight may be NULL)
 * (reference src/cpu_ref/rmsnorm_cpu.cpp:19-42). */
void orc_rmsnorm(const float* in, const float* weight, float* out, int64_t rows, int64_t cols,
                 float eps);

/* out = RMSNorm(in) . W[K x N] (reference src/cpu_ref/rmsnorm_linear_cpu.cpp:18-50). */
void orc_rmsnorm_linear(const float* in, const float* rms_weight, const float* W, float* out,
                        int64_t M, int64_t N, int64_t K, float eps);

/* As orc_rmsnorm_linear with a half weight matrix. */
void orc_rmsnorm_linear_f16w(const float* in, const float* rms_weight, const uint16_t* W,
                             float* out, int64_t M, int64_t N, int64_t K, float eps);

/* out[i] = a[i] + b[i] (reference src/cpu_ref/vector_add_cpu.cpp:8-12). */
void orc_vector_add(const float* a, const float* b, float* out, int64_t n);

/* sum = x + residual (float), written to sum_out when it is not NULL;
 * norm_out = sum / sqrt(mean(sum^2) + eps) * weight with the mean in double and
 * the scale rounded to float (reference src/cpu_ref/residual_rmsnorm_cpu.cpp:19-50).
 * residual, weight and sum_out may be NULL. */
void orc_residual_rmsnorm(const float* x, const float* residual, const float* weight,
                          float* norm_out, float* sum_out, int64_t rows, int64_t cols, float eps);

/* out[i] = g / (1 + exp(-g)) * u in double, rounded to float
 * (reference src/cpu_ref/swiglu_cpu.cpp:15-27). */
void orc_swiglu(const float* gate, const float* up, float* out, int64_t n);

/* Half gate / up / out, the same double formula, output rounded to half
 * (reference src/cpu_ref/swiglu_cpu.cpp:29-41). */
void orc_swiglu_fp16(const uint16_t* gate, const uint16_t* up, uint16_t* out, int64_t n);

/* act = swiglu(rmsnorm_linear(in, w, Wg), rmsnorm_linear(in, w, Wu)) with
 * Wg, Wu [K x N] (fp32, or half when the _f16w form): the gate / up projections
 * of a SwiGLU FFN, stated as the reference composes them (tests/test_kernels.cu:
 * 2900-2915: rmsnorm, matmul x2, swiglu). */
void orc_rmsnorm_linear_swiglu(const float* in, const float* rms_weight, const float* Wg,
                               const float* Wu, float* act, int64_t M, int64_t N, int64_t K,
                               float eps);
void orc_rmsnorm_linear_swiglu_f16w(const float* in, const float* rms_weight, const uint16_t* Wg,
                                    const uint16_t* Wu, float* act, int64_t M, int64_t N,
                                    int64_t K, float eps);

/* The SwiGLU FFN sub-block (reference tests/test_kernels.cu:2900-2915,
 * run_ffn_subblock_cpu): out = h + swiglu(n.Wg, n.Wu).Wd with n = rmsnorm(h, w);
 * h [S x D], Wg / Wu [D x F], Wd [F x D]. */
void orc_ffn_subblock(const float* h, const float* ffn_norm_w, const float* Wg, const float* Wu,
                      const float* Wd, float* out, int64_t S, int64_t D, int64_t F, float eps);

/* Multi-head / grouped-query attention with half q, k, v, out and a float64
 * two-pass softmax (reference src/cpu_ref/attention_cpu.cpp:84-155):
 * q / out [s_q, n_heads, head_dim]; k / v [n_kv_heads, kv_head_stride] with
 * key j of KV head h at h * kv_head_stride + j * head_dim; query head h reads
 * KV head h / (n_heads / n_kv_heads); causal rows see keys j <= q_pos_offset + i.
 * out_lse (may be NULL) receives m + log(sum exp) per row, -inf for an empty row.
 * Returns 0, or -1 when the arguments break the reference's preconditions
 * (nothing is written then). */
int orc_attention(const uint16_t* q, const uint16_t* k, const uint16_t* v, uint16_t* out,
                  int64_t s_q, int64_t s_kv, int64_t n_heads, int64_t n_kv_heads,
                  int64_t head_dim, int64_t kv_head_stride, float scale, int64_t q_pos_offset,
                  int is_causal, float* out_lse);

/* IEEE-754 binary16 conversions: half -> float exact; float -> half rounds to
 * nearest, ties to even (the rounding of the reference's CUDA build,
 * include/engine/half.hpp:28-32). */
float orc_half_to_float(uint16_t h);
uint16_t orc_float_to_half(float f);
void orc_f16_to_f32(const uint16_t* in, float* out, int64_t n);
void orc_f32_to_f16(const float* in, uint16_t* out, int64_t n);

/* Which planted mistake this build carries (0 = none). */
int orc_mutation(void);

#ifdef __cplusplus
}
#endif

#endif
