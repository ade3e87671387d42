/* rowwise_args.h -- kernel arguments of the row kernels (RMSNorm, residual +
 * RMSNorm, softmax, masked softmax), one layout for the device code
 * (rowwise_kernels.hpp) and for hosts that launch an emitted code object with
 * hipModuleLaunchKernel (csrc/runtime/launchers.cpp). */
#ifndef PK_ROWWISE_ARGS_H
#define PK_ROWWISE_ARGS_H

#include <stdint.h>

typedef struct pk_row_args {
  const void *in;         /* bf16 x [rows, cols] (RMSNorm, softmax) or fp32 logits (masked softmax) */
  const uint16_t *aux;    /* bf16 residual r (residual + RMSNorm) or additive mask (masked softmax) */
  const uint16_t *gamma;  /* bf16 [cols] RMSNorm weight or NULL */
  uint16_t *out;          /* bf16 [rows, cols] */
  int rows, cols;
  float inv_cols, eps;    /* RMSNorm: 1 / cols and epsilon */
} pk_row_args;

#endif /* PK_ROWWISE_ARGS_H */
