/* attention_args.h -- kernel arguments of the attention kernels, one layout
 * for the device code (attention_kernels.hpp) and for hosts that launch an
 * emitted code object with hipModuleLaunchKernel. */
#ifndef PK_ATTENTION_ARGS_H
#define PK_ATTENTION_ARGS_H

#include <stdint.h>

/* The generic kernel (any D <= 256). */
typedef struct pk_att_args {
  const uint16_t *Q, *K, *V;
  uint16_t *O;
  float *part_o;  /* [splits][BH][S_q][DP] when splits > 1 */
  float *part_ml; /* [splits][BH][S_q][2] */
  int BH, S_q, S_kv, D;
  int kv_rows;    /* rows per (b,h) in K/V storage (>= S_kv) */
  float scale;
  int causal;
  int splits;
  int q_tiles;
} pk_att_args;

/* The flash kernel (D 64 / 128). */
typedef struct pk_fa_args {
  const uint16_t *Q;
  const uint16_t *K, *V;    /* rows [0, S_cache) of each head, row stride D, head stride kv_rows */
  const uint16_t *Kn, *Vn;  /* fused append: rows [S_cache, S_kv) of each head (else null) */
  uint16_t *Kc, *Vc;        /* fused append: cache the new rows are copied into */
  uint16_t *O;
  float *part_o;            /* splits > 1: [splits][BH*S_q][DP] unnormalised */
  float *part_ml;           /* splits > 1: [splits][BH*S_q][2] (max, sum) */
  int BH, S_q, S_kv, S_cache, kv_rows;
  float scale;
  int causal;
  int q_tiles, splits;
} pk_fa_args;

/* In-place KV append: rows [S_cache, S_cache + S_new) of a cache holding
 * `cap` rows per (b,h). */
typedef struct pk_kv_append_args {
  uint16_t *cache;
  const uint16_t *neu;
  int64_t BH, S_cache, S_new, D, cap;
  int vec;  /* 16-byte copies (D % 8 == 0, aligned) */
} pk_kv_append_args;

#endif /* PK_ATTENTION_ARGS_H */
