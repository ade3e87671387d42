/*
 * polykernel_amd_runtime.h -- C-ABI of the runtime layer: tuning cache,
 * kernel cache, detect -> select -> serve, and the correctness-gated
 * autotuner.  The C++ API (polykernel_amd_runtime.hpp) is the primary
 * interface; these entry points expose it to C and to Python (ctypes).
 *
 * Conventions: return PK_OK (0) or a negative PK_ERR_* with the message in
 * pk_last_error(); calls that produce text (JSON documents, keys, hashes)
 * leave it in pk_last_text() -- valid until the next such call on the same
 * thread.  Shapes are the runtime's (M, N, K, dtype) keys.
 */
#ifndef POLYKERNEL_AMD_RUNTIME_H
#define POLYKERNEL_AMD_RUNTIME_H

#include <stddef.h>
#include <stdint.h>

#include "polykernel_amd.h"

#ifdef __cplusplus
extern "C" {
#endif

/* A cache miss, or an entry that is present but not validated. */
#define PK_ERR_NOT_FOUND -7

/* ---- argument blocks of the served ops (Runtime::Run's `io`) --------------
 * Device pointers; bf16 as raw uint16_t; `stream` a hipStream_t as void*. */
typedef struct pk_matmul_io { /* matmul, fused_matmul_bias_gelu, fused_matmul_bias_residual */
  const uint16_t *A, *B;
  uint16_t *C;
  const uint16_t *bias;     /* [N]: required by fused_matmul_bias_gelu, optional for *_residual */
  const uint16_t *residual; /* [M,N]: fused_matmul_bias_residual only */
  int M, N, K;
  void *stream;
} pk_matmul_io;

typedef struct pk_matmul_int8_io { /* matmul_int8, matmul_int8_gelu, matmul_int8_residual */
  const uint16_t *A;
  const int8_t *Wq;
  const float *scale;
  uint16_t *C;
  const uint16_t *residual; /* [M,N]: matmul_int8_residual only */
  int M, N, K;
  void *workspace; /* split partials; NULL = library-owned */
  size_t workspace_bytes;
  void *stream;
} pk_matmul_int8_io;

typedef struct pk_rmsnorm_matmul_io { /* fused_rmsnorm_matmul */
  const uint16_t *x, *gamma, *W; /* gamma may be NULL */
  uint16_t *out;
  int M, N, K;
  float eps;
  void *stream;
} pk_rmsnorm_matmul_io;

typedef struct pk_residual_rmsnorm_io { /* fused_residual_rmsnorm */
  const uint16_t *x, *r, *gamma; /* gamma may be NULL */
  uint16_t *out;
  int rows, cols;
  float eps;
  void *stream;
} pk_residual_rmsnorm_io;

typedef struct pk_softmax_mask_io { /* fused_softmax_mask */
  const float *logits;
  const uint16_t *mask;
  uint16_t *out;
  int rows, cols;
  void *stream;
} pk_softmax_mask_io;

typedef struct pk_kv_append_attention_io { /* fused_kv_append_attention */
  const uint16_t *Q;
  uint16_t *Kc, *Vc;
  const uint16_t *Kn, *Vn;
  uint16_t *O;
  int B, H, S_q, S_cache, D, cache_capacity;
  float scale;
  int causal;
  void *stream;
} pk_kv_append_attention_io;

/* Text result of the last call on this thread that produced one. */
PK_API const char *pk_last_text(void);

/* ---- tuning cache (KernelCache, lib/Runtime/KernelCache.h:38-157) -------- */
typedef struct pk_kernel_cache pk_kernel_cache;

PK_API pk_kernel_cache *pk_cache_create(void);
PK_API void pk_cache_destroy(pk_kernel_cache *cache);
/* Replace the entries with a tuning-cache document (tuning/schema.json). */
PK_API int pk_cache_load_tuning(pk_kernel_cache *cache, const char *json);
/* Add one entry given as a JSON object of the schema's entry form. */
PK_API int pk_cache_put(pk_kernel_cache *cache, const char *entry_json);
PK_API long long pk_cache_size(const pk_kernel_cache *cache);
/* The whole cache as a tuning-cache document -> pk_last_text(). */
PK_API int pk_cache_serialize(const pk_kernel_cache *cache);
/* Validated entry -> pk_last_text() as JSON; PK_ERR_NOT_FOUND on a miss or
 * an unvalidated entry (message in pk_last_error()). */
PK_API int pk_cache_select(const pk_kernel_cache *cache, const char *gpu, const char *op, long long M,
                           long long N, long long K, const char *dtype);
PK_API int pk_cache_put_binary(pk_kernel_cache *cache, const char *gpu, const char *op, long long M, long long N,
                               long long K, const char *dtype, const char *so_path, const char *kernel_hash);
/* {"so_path": ..., "kernel_hash": ...} -> pk_last_text(); PK_ERR_NOT_FOUND if none. */
PK_API int pk_cache_get_binary(const pk_kernel_cache *cache, const char *gpu, const char *op, long long M,
                               long long N, long long K, const char *dtype);
PK_API int pk_cache_persist(const pk_kernel_cache *cache, const char *dir);
PK_API int pk_cache_load_persisted(pk_kernel_cache *cache, const char *dir);
/* Number of entries dropped. */
PK_API long long pk_cache_invalidate_stale(pk_kernel_cache *cache);

/* FNV-1a 64 of a file -> pk_last_text() (16 hex digits). */
PK_API int pk_hash_file(const char *path);
/* "gpu/op/M=..,N=..,K=..,dtype" -> pk_last_text(). */
PK_API int pk_format_key(const char *gpu, const char *op, long long M, long long N, long long K,
                         const char *dtype);

/* ---- correctness gate (lib/Autotune/Benchmark.cpp:31-52) ----------------- */
PK_API int pk_passes_correctness_gate(double cosine, double max_rel_err, double pcc, double max_rel_ceiling);
PK_API double pk_rel_ceiling(const char *op, long long K);
/* Index of the fastest validated variant (ties: lowest index), -1 if none.
 * time_ms[i] is ignored where validated[i] == 0; NaN means "not timed". */
PK_API int pk_select_best_validated(const int *validated, const double *time_ms, int n);

/* ---- config space ------------------------------------------------------- */
/* ConfigSpace::Candidates as a JSON array of configs -> pk_last_text(). */
PK_API int pk_config_candidates(const char *op, long long M, long long N, long long K, const char *dtype);

/* ---- runtime (Runtime, lib/Runtime/Runtime.h:40-97) ---------------------- */
typedef struct pk_runtime pk_runtime;

/* A runtime over `cache` (which must outlive it) with every built-in op's
 * launcher registered.  fixed_arch NULL: detect the HIP device; otherwise a
 * fixed detector reporting that arch (for tests). */
PK_API pk_runtime *pk_runtime_create(const pk_kernel_cache *cache, const char *fixed_arch);
PK_API void pk_runtime_destroy(pk_runtime *rt);
/* As pk_runtime_create; with PK_RUNTIME_CODE_OBJECTS in `flags` every op is
 * served from the code object the cache holds for its entry
 * (pk_emit_code_object) instead of the linked kernels. */
#define PK_RUNTIME_CODE_OBJECTS 1
PK_API pk_runtime *pk_runtime_create_ex(const pk_kernel_cache *cache, const char *fixed_arch, int flags);
/* detect + select; the entry -> pk_last_text(). */
PK_API int pk_runtime_resolve(pk_runtime *rt, const char *op, long long M, long long N, long long K,
                              const char *dtype);
/* detect + select + serve; `io` points at the op's pk_*_io block. */
PK_API int pk_runtime_run(pk_runtime *rt, const char *op, long long M, long long N, long long K, const char *dtype,
                          void *io);

/* ---- emitter ------------------------------------------------------------------ */
/* The gfx950 HIP source of a tuned entry (JSON, schema entry form) ->
 * pk_last_text(); only the int8 ops are emitted. */
PK_API int pk_emit_source(const char *entry_json);
/* Emit + compile (hipcc --genco, child process) the entry's code object into
 * out_dir, then record the entry and the object's path and FNV-1a hash in
 * `cache`.  csrc_dir: the directory holding int8_stream.hpp. */
PK_API int pk_emit_code_object(pk_kernel_cache *cache, const char *entry_json, const char *csrc_dir,
                               const char *out_dir);

/* ---- autotuner ------------------------------------------------------------ */
/* Sweep (op, shape) on the current device.  options_json may be NULL or an
 * object with any of: warmup, iters, rounds, rotate_bytes, rel_ceiling,
 * max_variants, seed, batch_heads, verbose, inject_broken.  Result ->
 * pk_last_text(): {"entry": <schema entry>, "variants": [{"config", "name",
 * "validated", "time_ms", "model_violations", "correctness"}, ...]}. */
PK_API int pk_autotune(const char *op, long long M, long long N, long long K, const char *dtype,
                       const char *options_json);

#ifdef __cplusplus
}
#endif

#endif /* POLYKERNEL_AMD_RUNTIME_H */
