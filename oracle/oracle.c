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
 *   orc_vector_add        exact: a + b is one float rounding, compared bit for
 *                         bit with NumPy float32 addition.
 *   orc_residual_rmsnorm  golden vectors (RESIDUAL_RMSNORM_SHAPES), zeros give
 *                         zeros not NaN, NULL weight == ones, sum_out bit-exact
 *                         x + residual, equality with orc_rmsnorm of the sum;
 *                         planted dropped-residual mutation must be caught.
 *   orc_swiglu            golden vectors (SWIGLU_SIZES, NumPy float64 with the
 *                         overflow-safe sigmoid), closed forms silu(0) = 0,
 *                         up = 0 gives 0, silu(g) - silu(-g) == g, large |g|
 *                         limits; planted sign-flipped sigmoid must be caught.
 *   orc_swiglu_fp16       golden vectors with half output rounding, exact
 *                         agreement with orc_swiglu of the decoded halves
 *                         rounded to half.
 *   orc_rmsnorm_linear_swiglu(_f16w)  bit-exact equality with orc_rmsnorm_linear
 *                         (gate and up) followed by orc_swiglu.
 *   orc_ffn_subblock      golden vectors (FFN_SUBBLOCK_CASES), equality with the
 *                         composition of the pinned functions.
 *   orc_attention         golden vectors (the reference's ATTENTION_CASES decode
 *                         rows), closed forms (one key gives its value row,
 *                         q = 0 gives the mean of the value rows, a dominant
 *                         key gives its value row, key order does not matter),
 *                         NumPy float64 softmax on random heads; planted wrong
 *                         GQA head mapping must be caught.
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

/* ------------------------------------------------------ elementwise ops */

void orc_vector_add(const float* a, const float* b, float* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = a[i] + b[i];
}

void orc_residual_rmsnorm(const float* x, const float* residual, const float* weight,
                          float* norm_out, float* sum_out, int64_t rows, int64_t cols, float eps) {
  for (int64_t r = 0; r < rows; ++r) {
    const float* xr = x + r * cols;
    const float* rr = residual != NULL ? residual + r * cols : NULL;
    float* dn = norm_out + r * cols;
    float* ds = sum_out != NULL ? sum_out + r * cols : NULL;
    double sumsq = 0.0;
    for (int64_t c = 0; c < cols; ++c) {
#if ORC_MUTATION == 7
      /* planted mistake: the residual is not added */
      const float s = xr[c];
      (void)rr;
#else
      const float s = xr[c] + (rr != NULL ? rr[c] : 0.0f);
#endif
      if (ds != NULL) ds[c] = s;
      sumsq += (double)s * (double)s;
    }
    const float scale = (float)(1.0 / sqrt(sumsq / (double)cols + (double)eps));
    for (int64_t c = 0; c < cols; ++c) {
#if ORC_MUTATION == 7
      const float s = xr[c];
#else
      const float s = xr[c] + (rr != NULL ? rr[c] : 0.0f);
#endif
      const float w = weight != NULL ? weight[c] : 1.0f;
      dn[c] = s * scale * w;
    }
  }
}

static double silu64(double g) {
#if ORC_MUTATION == 6
  /* planted mistake: sigmoid with the wrong sign */
  return g / (1.0 + exp(g));
#else
  return g / (1.0 + exp(-g));
#endif
}

void orc_swiglu(const float* gate, const float* up, float* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = (float)(silu64((double)gate[i]) * (double)up[i]);
}

void orc_swiglu_fp16(const uint16_t* gate, const uint16_t* up, uint16_t* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) {
    const double g = (double)orc_half_to_float(gate[i]);
    const double u = (double)orc_half_to_float(up[i]);
    out[i] = orc_float_to_half((float)(silu64(g) * u));
  }
}

static void rmsnorm_linear_swiglu_any(const float* in, const float* rms_weight, const float* Wgf,
                                      const float* Wuf, const uint16_t* Wgh, const uint16_t* Wuh,
                                      float* act, int64_t M, int64_t N, int64_t K, float eps) {
  const size_t n = (size_t)(M > 0 ? M : 1) * (size_t)(N > 0 ? N : 1);
  float* gate = (float*)malloc(n * sizeof(float));
  float* up = (float*)malloc(n * sizeof(float));
  if (gate == NULL || up == NULL) abort();
  rmsnorm_linear_any(in, rms_weight, Wgf, Wgh, gate, M, N, K, eps);
  rmsnorm_linear_any(in, rms_weight, Wuf, Wuh, up, M, N, K, eps);
  orc_swiglu(gate, up, act, M * N);
  free(gate);
  free(up);
}

void orc_rmsnorm_linear_swiglu(const float* in, const float* rms_weight, const float* Wg,
                               const float* Wu, float* act, int64_t M, int64_t N, int64_t K,
                               float eps) {
  rmsnorm_linear_swiglu_any(in, rms_weight, Wg, Wu, NULL, NULL, act, M, N, K, eps);
}

void orc_rmsnorm_linear_swiglu_f16w(const float* in, const float* rms_weight, const uint16_t* Wg,
                                    const uint16_t* Wu, float* act, int64_t M, int64_t N,
                                    int64_t K, float eps) {
  rmsnorm_linear_swiglu_any(in, rms_weight, NULL, NULL, Wg, Wu, act, M, N, K, eps);
}

void orc_ffn_subblock(const float* h, const float* ffn_norm_w, const float* Wg, const float* Wu,
                      const float* Wd, float* out, int64_t S, int64_t D, int64_t F, float eps) {
  const size_t sd = (size_t)(S > 0 ? S : 1) * (size_t)(D > 0 ? D : 1);
  const size_t sf = (size_t)(S > 0 ? S : 1) * (size_t)(F > 0 ? F : 1);
  float* hn = (float*)malloc(sd * sizeof(float));
  float* gate = (float*)malloc(sf * sizeof(float));
  float* up = (float*)malloc(sf * sizeof(float));
  float* act = (float*)malloc(sf * sizeof(float));
  float* down = (float*)malloc(sd * sizeof(float));
  if (!hn || !gate || !up || !act || !down) abort();
  orc_rmsnorm(h, ffn_norm_w, hn, S, D, eps);
  orc_matmul(hn, Wg, gate, S, F, D);
  orc_matmul(hn, Wu, up, S, F, D);
  orc_swiglu(gate, up, act, S * F);
  orc_matmul(act, Wd, down, S, D, F);
  orc_vector_add(h, down, out, S * D);
  free(hn);
  free(gate);
  free(up);
  free(act);
  free(down);
}

/* ------------------------------------------------------------ attention */

int orc_attention(const uint16_t* q, const uint16_t* k, const uint16_t* v, uint16_t* out,
                  int64_t s_q, int64_t s_kv, int64_t n_heads, int64_t n_kv_heads,
                  int64_t head_dim, int64_t kv_head_stride, float scale, int64_t q_pos_offset,
                  int is_causal, float* out_lse) {
  if (q == NULL || k == NULL || v == NULL || out == NULL) return -1;
  if (s_q < 0 || s_kv < 0 || q_pos_offset < 0 || n_heads <= 0 || n_kv_heads <= 0) return -1;
  if (n_heads % n_kv_heads != 0 || (head_dim != 64 && head_dim != 128)) return -1;
  if (!isfinite(scale)) return -1;
  if (kv_head_stride < (s_kv > 0 ? s_kv * head_dim : 0)) return -1;
  const int64_t rows = s_q * n_heads;
  if (s_kv == 0) {
    for (int64_t i = 0; i < rows * head_dim; ++i) out[i] = 0;
    if (out_lse != NULL)
      for (int64_t r = 0; r < rows; ++r) out_lse[r] = -INFINITY;
    return 0;
  }
  const int64_t group = n_heads / n_kv_heads;
  double* scores = (double*)malloc((size_t)s_kv * sizeof(double));
  double* acc = (double*)malloc((size_t)head_dim * sizeof(double));
  if (scores == NULL || acc == NULL) abort();
  for (int64_t i = 0; i < s_q; ++i) {
    const int64_t last = is_causal ? (q_pos_offset + i < s_kv - 1 ? q_pos_offset + i : s_kv - 1)
                                   : s_kv - 1;
    for (int64_t h = 0; h < n_heads; ++h) {
      const int64_t row = i * n_heads + h;
      const uint16_t* qr = q + row * head_dim;
      uint16_t* orow = out + row * head_dim;
#if ORC_MUTATION == 8
      /* planted mistake: query head h reads KV head h % n_kv_heads */
      const int64_t hk = h % n_kv_heads;
      (void)group;
#else
      const int64_t hk = h / group;
#endif
      const uint16_t* kh = k + hk * kv_head_stride;
      const uint16_t* vh = v + hk * kv_head_stride;
      double m = -INFINITY;
      for (int64_t j = 0; j <= last; ++j) {
        double dot = 0.0;
        for (int64_t d = 0; d < head_dim; ++d)
          dot += (double)orc_half_to_float(qr[d]) * (double)orc_half_to_float(kh[j * head_dim + d]);
        scores[j] = dot * (double)scale;
        if (scores[j] > m) m = scores[j];
      }
      if (last < 0 || !(m > -INFINITY)) {
        for (int64_t d = 0; d < head_dim; ++d) orow[d] = 0;
        if (out_lse != NULL) out_lse[row] = -INFINITY;
        continue;
      }
      double sum = 0.0;
      for (int64_t d = 0; d < head_dim; ++d) acc[d] = 0.0;
      for (int64_t j = 0; j <= last; ++j) {
        const double w = exp(scores[j] - m);
        sum += w;
        for (int64_t d = 0; d < head_dim; ++d)
          acc[d] += w * (double)orc_half_to_float(vh[j * head_dim + d]);
      }
      const double inv = 1.0 / sum;
      for (int64_t d = 0; d < head_dim; ++d) orow[d] = orc_float_to_half((float)(acc[d] * inv));
      if (out_lse != NULL) out_lse[row] = (float)(m + log(sum));
    }
  }
  free(scores);
  free(acc);
  return 0;
}
