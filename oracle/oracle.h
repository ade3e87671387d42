/*
 * oracle.h -- CPU restatement of the PolyKernel reference arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the parity checker: only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it.  The
 * product (polykernel_amd) never links, loads or calls it.
 *
 * Rounding contract (kernels/cpu/cpu_reference.h:14-21 of the reference):
 *   bf16 inputs are exact fp32; every reduction accumulates in fp32 in the
 *   reference's sequential order (compiled with -ffp-contract=off so that
 *   `acc += a*b` keeps two roundings, as the reference's default x86-64 build
 *   does); each op's output is rounded back to bf16 (RNE).  Fused ops are the
 *   compositions of tests/golden/golden.py, so they round at every stage the
 *   golden rounds.
 *
 * All row loops are OpenMP-parallel over independent rows/columns; the order of
 * every individual reduction is the sequential one, so results do not depend
 * on the thread count.
 */
#ifndef PK_ORACLE_H
#define PK_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* kernels/cpu/cpu_reference.h:37-42 */
float pko_bf16_to_f32(uint16_t b);
/* kernels/cpu/cpu_reference.h:52-61 (RNE, NaN -> quiet NaN) */
uint16_t pko_f32_to_bf16(float f);
void pko_f32_to_bf16_array(const float *in, uint16_t *out, int64_t n);

/* kernels/cpu/cpu_reference.cpp:16-44 (weight may be NULL) */
void pko_rmsnorm(const uint16_t *in, const uint16_t *weight, uint16_t *out,
                 int64_t rows, int64_t cols, float eps);
/* tests/golden/golden.py:48-50 (same shapes, no broadcast) */
void pko_add(const uint16_t *a, const uint16_t *b, uint16_t *out, int64_t n);
/* tests/golden/golden.py:53-55 (bias[N] over rows of [M,N]) */
void pko_bias(const uint16_t *x, const uint16_t *bias, uint16_t *out, int64_t M, int64_t N);
/* tests/golden/golden.py:108-112 == rmsnorm(add(x, r), w, eps) */
void pko_residual_rmsnorm(const uint16_t *x, const uint16_t *r, const uint16_t *weight,
                          uint16_t *out, int64_t rows, int64_t cols, float eps);
/* kernels/cpu/cpu_reference.cpp:46-55 */
void pko_gelu(const uint16_t *in, uint16_t *out, int64_t n);
/* kernels/cpu/cpu_reference.cpp:64-78: c = bf16(sum_k a*b), k sequential */
void pko_matmul(const uint16_t *a, const uint16_t *b, uint16_t *c,
                int64_t M, int64_t N, int64_t K);
/* tests/golden/golden.py:96-100 (gamma may be NULL ==
 * kernels/cpu/cpu_reference.cpp:80-90) */
void pko_fused_rmsnorm_matmul(const uint16_t *x, const uint16_t *gamma, const uint16_t *w,
                              uint16_t *out, int64_t M, int64_t N, int64_t K, float eps);
/* kernels/cpu/cpu_reference.cpp:92-105 */
void pko_fused_matmul_bias_gelu(const uint16_t *a, const uint16_t *b, const uint16_t *bias,
                                uint16_t *out, int64_t M, int64_t N, int64_t K);
/* golden.add(golden.bias(golden.matmul(a, b), bias), residual); bias may be NULL
 * (then golden.add(golden.matmul(a, b), residual)) */
void pko_fused_matmul_bias_residual(const uint16_t *a, const uint16_t *b, const uint16_t *bias,
                                    const uint16_t *residual, uint16_t *out,
                                    int64_t M, int64_t N, int64_t K);
/* kernels/cpu/cpu_reference.cpp:107-128 */
void pko_softmax(const uint16_t *in, uint16_t *out, int64_t rows, int64_t cols);
/* tests/golden/golden.py:115-117 with fp32 logits: softmax(add(bf16(x), mask)) */
void pko_softmax_mask(const float *logits, const uint16_t *mask, uint16_t *out,
                      int64_t rows, int64_t cols);
/* kernels/cpu/attention.cpp:63-92 */
void pko_kv_append(const uint16_t *cache, const uint16_t *neu, uint16_t *out,
                   int64_t BH, int64_t S_cache, int64_t S_new, int64_t D);
/* kernels/cpu/attention.cpp:95-163 (scale passed in; the reference driver uses
 * 1.0f/sqrtf(D)) */
void pko_attention_prefill(const uint16_t *Q, const uint16_t *K, const uint16_t *V,
                           uint16_t *O, int64_t BH, int64_t S_q, int64_t S_kv,
                           int64_t D, float scale, int causal);
/* tests/golden/quant_golden.py:71-83 */
void pko_quantize_per_channel(const uint16_t *w, int8_t *wq, float *scale,
                              int64_t K, int64_t N);
/* kernels/cpu/matmul_quant.cpp:169-204 */
void pko_matmul_int8(const uint16_t *a, const int8_t *wq, const float *scale,
                     uint16_t *c, int64_t M, int64_t N, int64_t K);
/* Config-2 MLP block: add(bias(matmul(gelu(bias(matmul(rmsnorm(x,g),W1),b1)),W2),b2),x),
 * the chain of tests/e2e/test_mlp_correctness.py:117-126.  x:[M,d] W1:[d,F] W2:[F,d]. */
void pko_mlp_block(const uint16_t *x, const uint16_t *gamma, const uint16_t *w1,
                   const uint16_t *b1, const uint16_t *w2, const uint16_t *b2,
                   uint16_t *out, int64_t M, int64_t d, int64_t F, float eps);
/* Config-5 decode chain: add(matmul_int8(gelu(matmul_int8(x,W1q,s1)),W2q,s2), x) */
void pko_decode_mlp_int8(const uint16_t *x, const int8_t *w1q, const float *s1,
                         const int8_t *w2q, const float *s2, uint16_t *out,
                         int64_t M, int64_t d, int64_t F);

/* Number of OpenMP threads the oracle uses (1 when built without OpenMP). */
int pko_num_threads(void);
void pko_set_num_threads(int n);

#ifdef __cplusplus
}
#endif

#endif /* PK_ORACLE_H */
