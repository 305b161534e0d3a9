/*
 * oracle.c -- TEST INFRASTRUCTURE ONLY (see oracle.h). Never linked into the
 * engine; loaded by tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg.
 *
 * Each function restates the reference's scalar CPU oracle (file:line in
 * oracle.h). How each one is pinned (tests/test_oracle.py):
 *   orc_matmul            golden vectors (NumPy float64 A @ B over the
 *                         reference's MATMUL_SHAPES case table), A . I == A
 *                         exactly, all-ones product == K exactly, exact
 *                         rational brute force on tiny shapes, planted
 *                         transposed-B mutation must be caught.
 *   orc_gemv              golden vectors (GEMV_SHAPES), bit-exact equality with
 *                         orc_matmul at M = 1, x = 0 gives exact 0, planted
 *                         dropped-term mutation must be caught.
 *   orc_gemv_fp16         golden vectors (GEMV_FP16_SHAPES) with the half
 *                         output rounding in the bound, exact half outputs on
 *                         small-integer inputs.
 *   orc_gemv_f16w         golden vectors, equality with orc_gemv on the
 *                         half-decoded matrix.
 *   orc_rmsnorm           golden vectors (RMSNORM_SHAPES), zero row gives 0
 *                         not NaN, NULL weight == all-ones weight, planted
 *                         eps-outside-sqrt mutation must be caught.
 *   orc_rmsnorm_linear    golden vectors (RMSNORM_LINEAR_SHAPES), equality with
 *                         orc_rmsnorm followed by orc_matmul, NULL weight ==
 *                         ones, planted dropped-gain mutation must be caught.
 *   orc_rmsnorm_linear_f16w  equality with orc_rmsnorm_linear on the
 *                         half-decoded matrix.
 *   half conversions      all 65536 half -> float against NumPy float16,
 *                         float -> half against NumPy on 2^24 sampled floats
 *                         plus every boundary case; planted truncation
 *                         mutation must be caught.
 *
 * Build with -ffp-contract=off so `acc += a * b` is a multiply then an add in
 * double, as in the reference's scalar loops.
 */
#include "oracle.h"

#include <math.h>
#include <stddef.h>
#include <stdlib.h>
#include <string.h>

#ifndef ORC_MUTATION
#define ORC_MUTATION 0
#endif

int orc_mutation(void) { return ORC_MUTATION; }

/* ---------------------------------------------------------------- half */

float orc_half_to_float(uint16_t h) {
  const int sign = (h >> 15) & 1;
  const int exp = (h >> 10) & 0x1f;
  const int mant = h & 0x3ff;
  double v;
  if (exp == 0) {
    v = ldexp((double)mant, -24);
  } else if (exp == 31) {
    if (mant == 0) {
      v = INFINITY;
    } else {
      uint32_t bits = ((uint32_t)sign << 31) | 0x7f800000u | ((uint32_t)mant << 13);
      float f;
      memcpy(&f, &bits, sizeof f);
      return f;
    }
  } else {
    v = ldexp((double)(1024 + mant), exp - 25);
  }
  return (float)(sign ? -v : v);
}

uint16_t orc_float_to_half(float f) {
  uint32_t bits;
  memcpy(&bits, &f, sizeof bits);
  const uint16_t sign = (uint16_t)((bits >> 16) & 0x8000u);
  if (isnan(f)) return (uint16_t)(sign | 0x7e00u | ((bits >> 13) & 0x3ffu));
  if (isinf(f)) return (uint16_t)(sign | 0x7c00u);
  const double a = fabs((double)f);
  if (a == 0.0) return sign;
  int e2;
  (void)frexp(a, &e2);
  int E = e2 - 1; /* a in [2^E, 2^(E+1)) */
#if ORC_MUTATION == 5
  /* planted mistake: truncate instead of rounding to nearest even */
  if (E < -14) return (uint16_t)(sign | (uint16_t)floor(ldexp(a, 24)));
  {
    double m = floor(ldexp(a, 10 - E));
    if (E > 15) return (uint16_t)(sign | 0x7c00u);
    return (uint16_t)(sign | ((E + 15) << 10) | ((int)m - 1024));
  }
#else
  if (E < -14) {
    /* subnormal half: m * 2^-24, m = a * 2^24 rounded to nearest even (may reach 1024) */
    const double m = rint(ldexp(a, 24));
    return (uint16_t)(sign | (uint16_t)m);
  }
  double m = rint(ldexp(a, 10 - E)); /* in [1024, 2048] */
  if (m == 2048.0) {
    m = 1024.0;
    E += 1;
  }
  if (E > 15) return (uint16_t)(sign | 0x7c00u);
  return (uint16_t)(sign | ((E + 15) << 10) | ((int)m - 1024));
#endif
}

void orc_f16_to_f32(const uint16_t* in, float* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = orc_half_to_float(in[i]);
}

void orc_f32_to_f16(const float* in, uint16_t* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = orc_float_to_half(in[i]);
}

/* -------------------------------------------------------------- matmul */

void orc_matmul(const float* A, const float* B, float* C, int64_t M, int64_t N, int64_t K) {
  for (int64_t i = 0; i < M; ++i) {
    for (int64_t j = 0; j < N; ++j) {
      double acc = 0.0;
      for (int64_t k = 0; k < K; ++k) {
#if ORC_MUTATION == 1
        /* planted mistake: B read transposed */
        acc += (double)A[i * K + k] * (double)B[j * K + k];
#else
        acc += (double)A[i * K + k] * (double)B[k * N + j];
#endif
      }
      C[i * N + j] = (float)acc;
    }
  }
}

/* ---------------------------------------------------------------- gemv */

void orc_gemv(const float* A, const float* x, float* out, int64_t N, int64_t K) {
#if ORC_MUTATION == 2
  /* planted mistake: the last term of every dot product is dropped */
  const int64_t kend = K > 0 ? K - 1 : 0;
#else
  const int64_t kend = K;
#endif
  for (int64_t j = 0; j < N; ++j) {
    double acc = 0.0;
    for (int64_t k = 0; k < kend; ++k) acc += (double)x[k] * (double)A[k * N + j];
    out[j] = (float)acc;
  }
}

void orc_gemv_fp16(const uint16_t* A, const uint16_t* x, uint16_t* out, int64_t N, int64_t K) {
  for (int64_t j = 0; j < N; ++j) {
    double acc = 0.0;
    for (int64_t k = 0; k < K; ++k) {
      const double xk = (double)orc_half_to_float(x[k]);
      const double akj = (double)orc_half_to_float(A[k * N + j]);
      acc += xk * akj;
    }
    out[j] = orc_float_to_half((float)acc);
  }
}

void orc_gemv_f16w(const uint16_t* A, const float* x, float* out, int64_t N, int64_t K) {
  for (int64_t j = 0; j < N; ++j) {
    double acc = 0.0;
    for (int64_t k = 0; k < K; ++k) acc += (double)x[k] * (double)orc_half_to_float(A[k * N + j]);
    out[j] = (float)acc;
  }
}

/* ------------------------------------------------------------- rmsnorm */

static float row_scale(const float* src, int64_t cols, float eps) {
  double sumsq = 0.0;
  for (int64_t c = 0; c < cols; ++c) sumsq += (double)src[c] * (double)src[c];
  const double mean_sq = sumsq / (double)cols;
#if ORC_MUTATION == 3
  /* planted mistake: eps outside the square root */
  return (float)(1.0 / sqrt(mean_sq) + (double)eps);
#else
  return (float)(1.0 / sqrt(mean_sq + (double)eps));
#endif
}

void orc_rmsnorm(const float* in, const float* weight, float* out, int64_t rows, int64_t cols,
                 float eps) {
  for (int64_t r = 0; r < rows; ++r) {
    const float* src = in + r * cols;
    float* dst = out + r * cols;
    const float scale = row_scale(src, cols, eps);
    for (int64_t c = 0; c < cols; ++c) {
      const float w = weight != NULL ? weight[c] : 1.0f;
      dst[c] = src[c] * scale * w;
    }
  }
}

static void rmsnorm_linear_any(const float* in, const float* rms_weight, const float* Wf,
                               const uint16_t* Wh, float* out, int64_t M, int64_t N, int64_t K,
                               float eps) {
  float* temp = (float*)malloc((size_t)(K > 0 ? K : 1) * sizeof(float));
  if (temp == NULL) abort();
  for (int64_t r = 0; r < M; ++r) {
    const float* src = in + r * K;
    float* dst = out + r * N;
    const float scale = row_scale(src, K, eps);
    for (int64_t k = 0; k < K; ++k) {
#if ORC_MUTATION == 4
      /* planted mistake: the RMSNorm gain is ignored */
      const float w = 1.0f;
      (void)rms_weight;
#else
      const float w = rms_weight != NULL ? rms_weight[k] : 1.0f;
#endif
      temp[k] = src[k] * scale * w;
    }
    for (int64_t n = 0; n < N; ++n) {
      double acc = 0.0;
      for (int64_t k = 0; k < K; ++k) {
        const double wkn = Wf != NULL ? (double)Wf[k * N + n] : (double)orc_half_to_float(Wh[k * N + n]);
        acc += (double)temp[k] * wkn;
      }
      dst[n] = (float)acc;
    }
  }
  free(temp);
}

void orc_rmsnorm_linear(const float* in, const float* rms_weight, const float* W, float* out,
                        int64_t M, int64_t N, int64_t K, float eps) {
  rmsnorm_linear_any(in, rms_weight, W, NULL, out, M, N, K, eps);
}

void orc_rmsnorm_linear_f16w(const float* in, const float* rms_weight, const uint16_t* W,
                             float* out, int64_t M, int64_t N, int64_t K, float eps) {
  rmsnorm_linear_any(in, rms_weight, NULL, W, out, M, N, K, eps);
}
