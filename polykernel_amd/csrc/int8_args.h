/* int8_args.h -- kernel arguments of the streaming int8 kernel, one layout for
 * the device code (int8_stream.hpp) and for hosts that launch it from a code
 * object with hipModuleLaunchKernel (csrc/runtime/launchers.cpp). */
#ifndef PK_INT8_ARGS_H
#define PK_INT8_ARGS_H

#include <stdint.h>

typedef struct pk_i8s_args {
  const uint16_t *A;         /* bf16 [M, K] */
  const int8_t *W;           /* int8 [K, N] */
  const float *scale;        /* [N] */
  float *partial;            /* [splits][M][N] fp32 when splits > 1 */
  uint16_t *C;               /* bf16 [M, N] */
  const uint16_t *R;         /* bf16 [M, N] residual (epilogue 2) */
  const uint16_t *gelu_tab;  /* device GELU table (epilogue 1) */
  int M, N, K;
  int splits;       /* K splits per column slice */
  int split_steps;  /* 64-row steps per split */
  int units;        /* column slices * splits */
} pk_i8s_args;

/* Threads per workgroup of the split reduction (reduce8_body), for every host
 * that launches it: 8 outputs per thread, one grid-stride pass. */
#define PK_I8_REDUCE_THREADS 128

#endif /* PK_INT8_ARGS_H */
