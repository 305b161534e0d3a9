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
