/* gemm_args.h -- kernel arguments of the bf16 GEMM and RMSNorm -> MatMul
 * kernels, one layout for the device code (gemm_kernels.hpp) and for hosts
 * that launch an emitted code object with hipModuleLaunchKernel
 * (csrc/runtime/launchers.cpp). */
#ifndef PK_GEMM_ARGS_H
#define PK_GEMM_ARGS_H

#include <stdint.h>

typedef struct pk_gemm_args {
  const uint16_t *A;         /* bf16 [M, K] */
  const uint16_t *B;         /* bf16 [K, N] */
  uint16_t *C;               /* bf16 [M, N] */
  const uint16_t *bias;      /* bf16 [N] (epilogues 1 and 2) */
  const uint16_t *R;         /* bf16 [M, N] residual (epilogues 2 and 3) */
  const uint16_t *gelu_tab;  /* device GELU table (epilogue 1) */
  int M, N, K;
} pk_gemm_args;

/* RMSNorm -> MatMul panel kernels: out = bf16(bf16((x / rms) * gamma) @ W) */
typedef struct pk_panel_args {
  const uint16_t *X;      /* bf16 [M, K] */
  const uint16_t *gamma;  /* bf16 [K] or NULL */
  const uint16_t *B;      /* bf16 [K, N] */
  uint16_t *C;            /* bf16 [M, N] */
  int M, N, K;
  float inv_cols, eps;    /* 1 / K and the RMSNorm epsilon */
} pk_panel_args;

/* Launch geometry of the whole-K panel kernel (rmsnorm_panel_fast_body), for
 * every host that launches it: 8 waves per 32 x 64 output tile, and dynamic
 * LDS for the W slice (K x 64 bf16) and the normalised x panel (32 x K bf16),
 * at least the three fp32 32 x 64 partial tiles its K parts are summed
 * through at the end. */
#define PK_PANEL_THREADS 512
static inline unsigned pk_panel_lds_bytes(int K) {
  const unsigned need = (unsigned)K * 128u + 64u * (unsigned)K;
  return need > 24576u ? need : 24576u;
}

#endif /* PK_GEMM_ARGS_H */
