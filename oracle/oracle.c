/*
 * oracle.c -- CPU restatement of the PolyKernel reference arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY (the parity checker).  Loaded by tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg; never by the
 * product library.  Build: oracle/Makefile (gcc -O2 -ffp-contract=off -fopenmp).
 *
 * Each function cites the reference file:line whose arithmetic it follows.
 * Pinning (how each function is checked, besides this restatement):
 *   - bf16 conversion: on the host, a structured sweep (all 65536 upper
 *     halves x 10 rounding classes of the dropped bits) against torch's RNE
 *     conversion and the NaN rule (tests/test_oracle.py::
 *     test_bf16_rne_structured_sweep); the exhaustive 2^32 comparison runs on
 *     the device against the hardware conversion (tests/test_gpu_parity.py).
 *   - add / bias: a structured sweep (every exponent difference 0..26, both
 *     signs, all mantissa pairs, subnormals, overflow, +-0, +-inf, NaN, random
 *     pairs) against numpy fp32 addition + torch RNE
 *     (tests/test_oracle.py::test_add_matches_independent_bf16_add).
 *   - rmsnorm / gelu / matmul / softmax / fused_*: bit-exact against the
 *     reference's own kernels/cpu drivers compiled into oracle/_ref, plus the
 *     hand-computed known answers of tests/golden/test_golden_self.py.
 *   - attention prefill / kv append / int8 matmul: bit-exact against the
 *     reference's attention / matmul_quant drivers in oracle/_ref, plus
 *     closed-form cases (S_kv=1 -> O=V, K=0 -> O=mean(V), exact int sums).
 *   - quantize: closed-form properties (max|wq|=127, zero column, exact ties
 *     round half-even) -- the reference has no C++ quantizer.
 *   - residual_rmsnorm / softmax_mask / mlp_block / decode chain:
 *     compositions of the pinned primitives, checked against the _ref drivers
 *     chained stage by stage.
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

/* kernels/cpu/cpu_reference.h:37-42 */
float pko_bf16_to_f32(uint16_t b) {
  uint32_t u = (uint32_t)b << 16;
  float f;
  memcpy(&f, &u, sizeof f);
  return f;
}

/* kernels/cpu/cpu_reference.h:52-61 */
uint16_t pko_f32_to_bf16(float f) {
  uint32_t u;
  memcpy(&u, &f, sizeof u);
  if ((u & 0x7F800000u) == 0x7F800000u && (u & 0x007FFFFFu) != 0u)
    return (uint16_t)((u >> 16) | 0x0040u);
  uint32_t lsb = (u >> 16) & 1u;
  u += 0x7FFFu + lsb;
  return (uint16_t)(u >> 16);
}

#define BF(x) pko_bf16_to_f32(x)
#define TOBF(x) pko_f32_to_bf16(x)

void pko_f32_to_bf16_array(const float *in, uint16_t *out, int64_t n) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; ++i) out[i] = TOBF(in[i]);
}

int pko_num_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

void pko_set_num_threads(int n) {
#ifdef _OPENMP
  if (n > 0) omp_set_num_threads(n);
#else
  (void)n;
#endif
}

/* One row of kernels/cpu/cpu_reference.cpp:16-44. */
static void rmsnorm_row(const uint16_t *x, const uint16_t *w, uint16_t *y,
                        int64_t cols, float inv_cols, float eps) {
  float sum_sq = 0.0f;
  for (int64_t i = 0; i < cols; ++i) {
    float v = BF(x[i]);
    sum_sq += v * v;
  }
  float rms = sqrtf(sum_sq * inv_cols + eps);
  for (int64_t i = 0; i < cols; ++i) {
    float v = BF(x[i]) / rms;
    if (w) v *= BF(w[i]);
    y[i] = TOBF(v);
  }
}

void pko_rmsnorm(const uint16_t *in, const uint16_t *weight, uint16_t *out,
                 int64_t rows, int64_t cols, float eps) {
  const float inv_cols = 1.0f / (float)cols;
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r)
    rmsnorm_row(in + r * cols, weight, out + r * cols, cols, inv_cols, eps);
}

/* tests/golden/golden.py:48-50 */
void pko_add(const uint16_t *a, const uint16_t *b, uint16_t *out, int64_t n) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; ++i) out[i] = TOBF(BF(a[i]) + BF(b[i]));
}

/* tests/golden/golden.py:53-55 */
void pko_bias(const uint16_t *x, const uint16_t *bias, uint16_t *out, int64_t M, int64_t N) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < M; ++i)
    for (int64_t j = 0; j < N; ++j) out[i * N + j] = TOBF(BF(x[i * N + j]) + BF(bias[j]));
}

/* tests/golden/golden.py:108-112: the sum is rounded to bf16 before the norm. */
void pko_residual_rmsnorm(const uint16_t *x, const uint16_t *r, const uint16_t *weight,
                          uint16_t *out, int64_t rows, int64_t cols, float eps) {
  const float inv_cols = 1.0f / (float)cols;
#pragma omp parallel
  {
    uint16_t *s = (uint16_t *)malloc((size_t)cols * sizeof(uint16_t));
#pragma omp for schedule(static)
    for (int64_t row = 0; row < rows; ++row) {
      const uint16_t *xr = x + row * cols, *rr = r + row * cols;
      for (int64_t i = 0; i < cols; ++i) s[i] = TOBF(BF(xr[i]) + BF(rr[i]));
      rmsnorm_row(s, weight, out + row * cols, cols, inv_cols, eps);
    }
    free(s);
  }
}

/* kernels/cpu/cpu_reference.cpp:46-55: erf in double on the fp32 product
 * x*0.70710678f, rounded to float; the outer (0.5f*x)*(1.0f+e) stays fp32. */
static inline uint16_t gelu_one(uint16_t xb) {
  const float kInvSqrt2 = 0.70710678118654752440f;
  float x = BF(xb);
  float e = (float)erf((double)(x * kInvSqrt2));
  return TOBF(0.5f * x * (1.0f + e));
}

void pko_gelu(const uint16_t *in, uint16_t *out, int64_t n) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; ++i) out[i] = gelu_one(in[i]);
}

/* kernels/cpu/cpu_reference.cpp:64-78.  The reference loops i,j,k with a
 * scalar accumulator; here the j loop is innermost over an fp32 accumulator
 * row, which performs for every (i,j) the identical sequence of roundings
 * (acc = acc + a[i][k]*b[k][j] for k = 0..K-1), so the bits are the same while
 * B is read row-contiguously. */
void pko_matmul(const uint16_t *a, const uint16_t *b, uint16_t *c,
                int64_t M, int64_t N, int64_t K) {
#pragma omp parallel
  {
    float *acc = (float *)malloc((size_t)N * sizeof(float));
    float *brow = (float *)malloc((size_t)N * sizeof(float));
#pragma omp for schedule(static)
    for (int64_t i = 0; i < M; ++i) {
      for (int64_t j = 0; j < N; ++j) acc[j] = 0.0f;
      const uint16_t *arow = a + i * K;
      for (int64_t k = 0; k < K; ++k) {
        const float av = BF(arow[k]);
        const uint16_t *bk = b + k * N;
        for (int64_t j = 0; j < N; ++j) brow[j] = BF(bk[j]);
        for (int64_t j = 0; j < N; ++j) acc[j] += av * brow[j];
      }
      for (int64_t j = 0; j < N; ++j) c[i * N + j] = TOBF(acc[j]);
    }
    free(acc);
    free(brow);
  }
}

/* tests/golden/golden.py:96-100 (matmul(rmsnorm(x, gamma, eps), w)). */
void pko_fused_rmsnorm_matmul(const uint16_t *x, const uint16_t *gamma, const uint16_t *w,
                              uint16_t *out, int64_t M, int64_t N, int64_t K, float eps) {
  uint16_t *normed = (uint16_t *)malloc((size_t)(M * K) * sizeof(uint16_t));
  pko_rmsnorm(x, gamma, normed, M, K, eps);
  pko_matmul(normed, w, out, M, N, K);
  free(normed);
}

/* kernels/cpu/cpu_reference.cpp:92-105 */
void pko_fused_matmul_bias_gelu(const uint16_t *a, const uint16_t *b, const uint16_t *bias,
                                uint16_t *out, int64_t M, int64_t N, int64_t K) {
  uint16_t *mm = (uint16_t *)malloc((size_t)(M * N) * sizeof(uint16_t));
  pko_matmul(a, b, mm, M, N, K);
  pko_bias(mm, bias, mm, M, N);
  pko_gelu(mm, out, M * N);
  free(mm);
}

/* golden add(bias(matmul(a, b), bias), residual): tests/golden/golden.py:48-60 */
void pko_fused_matmul_bias_residual(const uint16_t *a, const uint16_t *b, const uint16_t *bias,
                                    const uint16_t *residual, uint16_t *out,
                                    int64_t M, int64_t N, int64_t K) {
  uint16_t *mm = (uint16_t *)malloc((size_t)(M * N) * sizeof(uint16_t));
  pko_matmul(a, b, mm, M, N, K);
  if (bias) pko_bias(mm, bias, mm, M, N);
  pko_add(mm, residual, out, M * N);
  free(mm);
}

/* One row of kernels/cpu/cpu_reference.cpp:107-128 (max seeded from x[0] with
 * std::max semantics; exp evaluated again in the normalise pass). */
static void softmax_row(const uint16_t *x, uint16_t *y, int64_t cols) {
  float m = BF(x[0]);
  for (int64_t i = 1; i < cols; ++i) {
    float v = BF(x[i]);
    m = (m < v) ? v : m;
  }
  float sum = 0.0f;
  for (int64_t i = 0; i < cols; ++i) sum += expf(BF(x[i]) - m);
  float inv_sum = 1.0f / sum;
  for (int64_t i = 0; i < cols; ++i) y[i] = TOBF(expf(BF(x[i]) - m) * inv_sum);
}

void pko_softmax(const uint16_t *in, uint16_t *out, int64_t rows, int64_t cols) {
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r) softmax_row(in + r * cols, out + r * cols, cols);
}

/* tests/golden/golden.py:115-117: softmax(add(x, mask)); add rounds both
 * operands to bf16 first (golden.py:48-50), so fp32 logits are RNE'd. */
void pko_softmax_mask(const float *logits, const uint16_t *mask, uint16_t *out,
                      int64_t rows, int64_t cols) {
#pragma omp parallel
  {
    uint16_t *z = (uint16_t *)malloc((size_t)cols * sizeof(uint16_t));
#pragma omp for schedule(static)
    for (int64_t r = 0; r < rows; ++r) {
      for (int64_t i = 0; i < cols; ++i)
        z[i] = TOBF(BF(TOBF(logits[r * cols + i])) + BF(mask[r * cols + i]));
      softmax_row(z, out + r * cols, cols);
    }
    free(z);
  }
}

/* kernels/cpu/attention.cpp:63-92 */
void pko_kv_append(const uint16_t *cache, const uint16_t *neu, uint16_t *out,
                   int64_t BH, int64_t S_cache, int64_t S_new, int64_t D) {
#pragma omp parallel for schedule(static)
  for (int64_t bh = 0; bh < BH; ++bh) {
    uint16_t *o = out + bh * (S_cache + S_new) * D;
    memcpy(o, cache + bh * S_cache * D, (size_t)(S_cache * D) * sizeof(uint16_t));
    memcpy(o + S_cache * D, neu + bh * S_new * D, (size_t)(S_new * D) * sizeof(uint16_t));
  }
}

/* kernels/cpu/attention.cpp:95-163: per (bh, i): limit = S_kv - S_q + i under
 * the causal mask; score = (sequential q.k) * scale; max; w = exp(score - m)
 * with the sequential sum; o_d = bf16((sum_j w_j v_jd) * (1/sum)). */
void pko_attention_prefill(const uint16_t *Q, const uint16_t *K, const uint16_t *V,
                           uint16_t *O, int64_t BH, int64_t S_q, int64_t S_kv,
                           int64_t D, float scale, int causal) {
#pragma omp parallel
  {
    float *score = (float *)malloc((size_t)S_kv * sizeof(float));
    float *acc = (float *)malloc((size_t)D * sizeof(float));
#pragma omp for schedule(static) collapse(2)
    for (int64_t bh = 0; bh < BH; ++bh) {
      for (int64_t i = 0; i < S_q; ++i) {
        const uint16_t *q = Q + (bh * S_q + i) * D;
        const uint16_t *k = K + bh * S_kv * D;
        const uint16_t *v = V + bh * S_kv * D;
        const int64_t limit = causal ? (S_kv - S_q + i) : (S_kv - 1);
        float m = -HUGE_VALF;
        for (int64_t j = 0; j < S_kv; ++j) {
          if (j > limit) {
            score[j] = -HUGE_VALF;
            continue;
          }
          float dot = 0.0f;
          for (int64_t d = 0; d < D; ++d) dot += BF(q[d]) * BF(k[j * D + d]);
          score[j] = dot * scale;
          m = (m < score[j]) ? score[j] : m;
        }
        float sum = 0.0f;
        for (int64_t j = 0; j < S_kv; ++j) {
          score[j] = expf(score[j] - m);
          sum += score[j];
        }
        const float inv = 1.0f / sum;
        /* d-outer / j-inner in the reference; j-outer here keeps each
         * acc[d] = acc[d] + w_j*v_jd in increasing j, the same roundings. */
        for (int64_t d = 0; d < D; ++d) acc[d] = 0.0f;
        for (int64_t j = 0; j < S_kv; ++j) {
          const float w = score[j];
          const uint16_t *vj = v + j * D;
          for (int64_t d = 0; d < D; ++d) acc[d] += w * BF(vj[d]);
        }
        uint16_t *o = O + (bh * S_q + i) * D;
        for (int64_t d = 0; d < D; ++d) o[d] = TOBF(acc[d] * inv);
      }
    }
    free(score);
    free(acc);
  }
}

/* tests/golden/quant_golden.py:71-83.  amax/127 and wf/scale are fp32
 * divisions (numpy float32 arithmetic); np.rint is round-half-even, which is
 * nearbyintf under the default rounding mode. */
void pko_quantize_per_channel(const uint16_t *w, int8_t *wq, float *scale,
                              int64_t K, int64_t N) {
  /* amax per column (a max is exact in any order; rows outer keeps reads
   * contiguous), then scale = amax > 0 ? amax / 127 : 1. */
#pragma omp parallel for schedule(static)
  for (int64_t n0 = 0; n0 < N; n0 += 1024) {
    const int64_t n1 = (n0 + 1024 < N) ? n0 + 1024 : N;
    float amax[1024];
    for (int64_t n = n0; n < n1; ++n) amax[n - n0] = 0.0f;
    for (int64_t k = 0; k < K; ++k)
      for (int64_t n = n0; n < n1; ++n) {
        float a = fabsf(BF(w[k * N + n]));
        amax[n - n0] = (a > amax[n - n0]) ? a : amax[n - n0];
      }
    for (int64_t n = n0; n < n1; ++n)
      scale[n] = (amax[n - n0] > 0.0f) ? amax[n - n0] / 127.0f : 1.0f;
  }
#pragma omp parallel for schedule(static)
  for (int64_t k = 0; k < K; ++k) {
    for (int64_t n = 0; n < N; ++n) {
      float q = nearbyintf(BF(w[k * N + n]) / scale[n]);
      if (q > 127.0f) q = 127.0f;
      if (q < -127.0f) q = -127.0f;
      wq[k * N + n] = (int8_t)q;
    }
  }
}

/* kernels/cpu/matmul_quant.cpp:189-199: acc += a * (float(wq) * s), sequential k.
 * Same accumulator-row restructuring as pko_matmul (identical roundings). */
void pko_matmul_int8(const uint16_t *a, const int8_t *wq, const float *scale,
                     uint16_t *c, int64_t M, int64_t N, int64_t K) {
#pragma omp parallel
  {
    float *acc = (float *)malloc((size_t)N * sizeof(float));
    float *wrow = (float *)malloc((size_t)N * sizeof(float));
#pragma omp for schedule(static)
    for (int64_t i = 0; i < M; ++i) {
      for (int64_t j = 0; j < N; ++j) acc[j] = 0.0f;
      for (int64_t k = 0; k < K; ++k) {
        const float av = BF(a[i * K + k]);
        const int8_t *wk = wq + k * N;
        for (int64_t j = 0; j < N; ++j) wrow[j] = (float)wk[j] * scale[j];
        for (int64_t j = 0; j < N; ++j) acc[j] += av * wrow[j];
      }
      for (int64_t j = 0; j < N; ++j) c[i * N + j] = TOBF(acc[j]);
    }
    free(acc);
    free(wrow);
  }
}

void pko_mlp_block(const uint16_t *x, const uint16_t *gamma, const uint16_t *w1,
                   const uint16_t *b1, const uint16_t *w2, const uint16_t *b2,
                   uint16_t *out, int64_t M, int64_t d, int64_t F, float eps) {
  uint16_t *a = (uint16_t *)malloc((size_t)(M * d) * sizeof(uint16_t));
  uint16_t *h = (uint16_t *)malloc((size_t)(M * F) * sizeof(uint16_t));
  pko_rmsnorm(x, gamma, a, M, d, eps);
  pko_fused_matmul_bias_gelu(a, w1, b1, h, M, F, d);
  pko_fused_matmul_bias_residual(h, w2, b2, x, out, M, d, F);
  free(a);
  free(h);
}

void pko_decode_mlp_int8(const uint16_t *x, const int8_t *w1q, const float *s1,
                         const int8_t *w2q, const float *s2, uint16_t *out,
                         int64_t M, int64_t d, int64_t F) {
  uint16_t *t = (uint16_t *)malloc((size_t)(M * F) * sizeof(uint16_t));
  uint16_t *y = (uint16_t *)malloc((size_t)(M * d) * sizeof(uint16_t));
  pko_matmul_int8(x, w1q, s1, t, M, F, d);
  pko_gelu(t, t, M * F);
  pko_matmul_int8(t, w2q, s2, y, M, d, F);
  pko_add(y, x, out, M * d);
  free(t);
  free(y);
}
