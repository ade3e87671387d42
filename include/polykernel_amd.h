/*
 * polykernel_amd.h -- C-ABI of the MI355X (gfx950) fused transformer-block
 * kernels.  Drop-in for the reference's launch_* host entry points.
 *
 * Conventions (all entry points):
 *   - bf16 tensors travel as raw uint16_t bits (RNE), row-major, leading dims
 *     flattened by the caller; weight matrices are [K, N] with N contiguous,
 *     exactly the reference layouts (no hidden pre-pack).
 *   - Every pointer is a device pointer the caller allocated; launchers never
 *     allocate or free, except the few entry points whose reference signature
 *     has no workspace argument (marked "library workspace" below): those keep
 *     one lazily grown per-device buffer owned by the library.
 *   - `stream` is a hipStream_t passed as void* (NULL = the null stream); every
 *     launch is asynchronous on it.
 *   - Return value: PK_OK (0) on success, a negative PK_ERR_* otherwise; the
 *     message is available from pk_last_error() (thread-local).  Nothing in the
 *     library aborts the process.
 */
#ifndef POLYKERNEL_AMD_H
#define POLYKERNEL_AMD_H

#include <stddef.h>
#include <stdint.h>

#if defined(__GNUC__) || defined(__clang__)
#define PK_API __attribute__((visibility("default")))
#else
#define PK_API
#endif

#ifdef __cplusplus
extern "C" {
#endif

#define PK_OK 0
#define PK_ERR_INVALID_ARG -1
#define PK_ERR_LAUNCH -2
#define PK_ERR_WORKSPACE -3
#define PK_ERR_NO_DEVICE -4
#define PK_ERR_UNSUPPORTED -5
#define PK_ERR_HIP -6

/* ---- library / device -------------------------------------------------- */

/* Library version string, e.g. "polykernel_amd 0.1.0 gfx950". */
PK_API const char *pk_version(void);
/* Message of the last failing call on this thread ("" if none). */
PK_API const char *pk_last_error(void);
/* Optional eager set-up of the current device (GELU table); every launcher
 * also does it lazily on first use. */
PK_API int pk_init(void);
/* Bare gfx token of device `ordinal` ("gfx950"), written to buf.  Mirrors
 * lib/Runtime/DeviceDetect.cpp:28-50 + 79-84 of the reference. */
PK_API int pk_device_arch(int ordinal, char *buf, int buf_len);
/* Parse a raw gcnArchName ("gfx950:sramecc+:xnack-") into its gfx token.
 * Mirrors ParseGcnArchName, lib/Runtime/DeviceDetect.cpp:28-50. */
PK_API int pk_parse_gcn_arch_name(const char *gcn_arch_name, char *buf, int buf_len);

/* Device self-check: counts the fp32 inputs (all 2^32) on which the kernels'
 * fp32 -> bf16 conversion differs from the reference RNE formula
 * (kernels/cpu/cpu_reference.h:52-61).  Synchronous; allocates 8 bytes. */
PK_API int pk_check_bf16_conversion(unsigned long long *mismatches);
/* Device self-check of the two-codes-per-register GELU the GEMM epilogue
 * uses: counts the pairs (every low code x four high-code patterns) where it
 * differs from the per-element exact GELU.  Synchronous; allocates 8 bytes. */
PK_API int pk_check_gelu_pairs(unsigned long long *mismatches);

/* Self-check of the row kernels' division x / d (d the row's RMS): for each of
 * the n divisors (n <= 32768) and every bf16 numerator x inside the fast
 * path's range, counts the outputs that differ from the device's IEEE
 * division; and, for every bf16 code, counts a disagreement between the packed
 * magnitude range test and the float one.  Expected 0. */
PK_API int pk_check_row_division(const float *divisors, int n, unsigned long long *mismatches);

/* ---- reference entry points (same names and argument order) ------------ */

/* y = bf16(x / sqrt(mean(x^2) + eps) [* w]); w may be NULL.
 * Replaces launch_rmsnorm, kernels/generated/rmsnorm.cu:106-108. */
PK_API int launch_rmsnorm(const uint16_t *input, const uint16_t *weight, uint16_t *output,
                   int rows, int cols, float eps, void *stream);

/* Exact erf GELU, bit-exact with kernels/cpu/cpu_reference.cpp:46-55.
 * Replaces launch_gelu, kernels/generated/gelu.cu:56. */
PK_API int launch_gelu(const uint16_t *input, uint16_t *output, int n, void *stream);

/* C[M,N] = bf16(A[M,K] @ B[K,N]), fp32 accumulate on bf16 MFMA.
 * Replaces launch_matmul, kernels/generated/matmul.cu:78-79. */
PK_API int launch_matmul(const uint16_t *A, const uint16_t *B, uint16_t *C, int M, int N, int K,
                  void *stream);

/* Row softmax over the last axis.
 * Replaces launch_softmax, kernels/generated/softmax.cu:119-120. */
PK_API int launch_softmax(const uint16_t *input, uint16_t *output, int rows, int cols, void *stream);

/* out = matmul(rmsnorm(input, eps), weight), no gamma.
 * Replaces launch_fused_rmsnorm_matmul, kernels/generated/fused_rmsnorm_matmul.cu:114-116.
 * The normalised 32-row panel stays in LDS (the whole-K panel kernel) when
 * K % 64 == 0, K <= 832, N % 8 == 0, the operands are 16-byte aligned and the
 * grid is one round of at most 256 tiles of 32 x 64; otherwise the rows are
 * normalised once into library workspace and the GEMM reads them. */
PK_API int launch_fused_rmsnorm_matmul(const uint16_t *input, const uint16_t *weight, uint16_t *output,
                                int M, int N, int K, float eps, void *stream);

/* out = gelu(bias(matmul(a, b), bias)), per-stage bf16 as the reference.
 * Replaces launch_fused_matmul_bias_gelu, kernels/generated/fused_matmul_bias_gelu.cu:104-106. */
PK_API int launch_fused_matmul_bias_gelu(const uint16_t *a, const uint16_t *b, const uint16_t *bias,
                                  uint16_t *output, int M, int N, int K, void *stream);

/* Causal/non-causal SDPA, Q [B,H,S_q,D], K/V [B,H,S_kv,D], O [B,H,S_q,D],
 * any D <= 1024 (larger: PK_ERR_UNSUPPORTED).
 * Query i attends to keys j <= S_kv - S_q + i when causal.
 * Replaces launch_attention_prefill, kernels/generated/attention_prefill.cu:169-172. */
PK_API int launch_attention_prefill(const uint16_t *Q, const uint16_t *K, const uint16_t *V, uint16_t *O,
                             int B, int H, int S_q, int S_kv, int D, float scale, int causal,
                             void *stream);

/* out [B,H,S_cache+S_new,D] = concat(cache, new_rows) along the sequence axis.
 * Replaces launch_kv_cache_update, kernels/generated/kv_cache_update.cu:67-69. */
PK_API int launch_kv_cache_update(const uint16_t *cache, const uint16_t *new_rows, uint16_t *out, int B,
                           int H, int S_cache, int S_new, int D, void *stream);

/* C = bf16(A @ dequant(Wq, scale)), A bf16 [M,K], Wq int8 [K,N], scale fp32 [N].
 * Replaces launch_matmul_int8, kernels/generated/matmul_int8.cu:97-98.
 * Library workspace (split-K partials) for long-K decode shapes. */
PK_API int launch_matmul_int8(const uint16_t *A, const int8_t *Wq, const float *scale, uint16_t *C,
                       int M, int N, int K, void *stream);

/* launch_matmul_int8 without any allocation.  No counterpart in the
 * reference: for callers that cannot allocate device memory (code under HIP
 * graph capture, tight decode/serving loops, harnesses that forbid
 * hipMalloc).  Same arguments, kernels and results (bit-identical) as
 * launch_matmul_int8; the split-K partials live in a static 16 MiB device
 * array of the library (one per GPU, held until the process ends) instead of
 * the library workspace.  A shape whose split-K partials need more than
 * 16 MiB returns PK_ERR_WORKSPACE without launching.  Calls allocate nothing
 * (no hipMalloc / hipFree) and share the array: calls that overlap on one
 * GPU -- on any streams, from any threads -- race on it and must be
 * serialised by the caller.  pk_init() looks up the array's address for the
 * current device; otherwise the first call on a device does. */
PK_API int launch_matmul_int8_noalloc(const uint16_t *A, const int8_t *Wq, const float *scale, uint16_t *C,
                                      int M, int N, int K, void *stream);

/* ---- fused ops the reference has only as golden compositions ----------- */

/* out = rmsnorm(bf16(x + r), gamma, eps); gamma may be NULL.
 * tests/golden/golden.py:108-112; IR op PolyKernelOps.td:336-346. */
PK_API int launch_fused_residual_rmsnorm(const uint16_t *x, const uint16_t *r, const uint16_t *gamma,
                                  uint16_t *out, int rows, int cols, float eps, void *stream);

/* out = softmax(bf16(bf16(logits) + mask)), logits fp32, mask bf16 additive
 * (0 / -inf), same shape.  tests/golden/golden.py:115-117. */
PK_API int launch_fused_softmax_mask(const float *logits, const uint16_t *mask, uint16_t *out, int rows,
                              int cols, void *stream);

/* out = matmul(rmsnorm(x, gamma, eps), W); gamma may be NULL.
 * tests/golden/golden.py:96-100.  Same LDS / library-workspace rule. */
PK_API int launch_fused_rmsnorm_matmul_gamma(const uint16_t *x, const uint16_t *gamma, const uint16_t *W,
                                      uint16_t *out, int M, int N, int K, float eps, void *stream);

/* out = add(bias(matmul(a, b), bias), residual); bias may be NULL.
 * Chain of tests/e2e/test_mlp_correctness.py:117-126 (golden.py:48-60). */
PK_API int launch_fused_matmul_bias_residual(const uint16_t *a, const uint16_t *b, const uint16_t *bias,
                                      const uint16_t *residual, uint16_t *out, int M, int N, int K,
                                      void *stream);

/* In-place KV append + causal prefill.  Kc/Vc hold S_cache valid rows per
 * (b,h) with room for `cache_capacity` rows; Kn/Vn [B,H,S_q,D] are written at
 * rows [S_cache, S_cache+S_q) and attention runs over S_kv = S_cache + S_q.
 * golden fused_kv_append_attention, tests/golden/golden.py:139-172. */
PK_API int launch_fused_kv_append_attention(const uint16_t *Q, uint16_t *Kc, uint16_t *Vc,
                                     const uint16_t *Kn, const uint16_t *Vn, uint16_t *O, int B,
                                     int H, int S_q, int S_cache, int D, int cache_capacity,
                                     float scale, int causal, void *stream);

/* Symmetric per-output-channel int8 quantisation of bf16 W [K,N]; bit-exact
 * with tests/golden/quant_golden.py:71-83. */
PK_API int launch_quantize_int8_per_channel(const uint16_t *W, int8_t *Wq, float *scale, int K, int N,
                                     void *stream);

/* Config-2 MLP block: y = add(bias(matmul(gelu(bias(matmul(rmsnorm(x, gamma),
 * W1), b1)), W2), b2), x).  x [M,d], W1 [d,F], W2 [F,d].  `workspace` must
 * hold pk_mlp_block_workspace_size(M, d, F) bytes. */
PK_API size_t pk_mlp_block_workspace_size(int M, int d, int F);
PK_API int launch_mlp_block(const uint16_t *x, const uint16_t *gamma, const uint16_t *W1,
                     const uint16_t *b1, const uint16_t *W2, const uint16_t *b2, uint16_t *out,
                     int M, int d, int F, float eps, void *workspace, size_t workspace_bytes,
                     void *stream);

/* Config-5 int8 decode MLP: y = add(matmul_int8(gelu(matmul_int8(x, W1q, s1)),
 * W2q, s2), x).  `workspace` must hold pk_decode_mlp_int8_workspace_size bytes. */
PK_API size_t pk_decode_mlp_int8_workspace_size(int M, int d, int F);
PK_API int launch_decode_mlp_int8(const uint16_t *x, const int8_t *W1q, const float *s1,
                           const int8_t *W2q, const float *s2, uint16_t *out, int M, int d, int F,
                           void *workspace, size_t workspace_bytes, void *stream);

/* Tuning/test hook: one GEMM with an explicit epilogue (0 none, 1 bias+GELU,
 * 2 bias+residual, 3 residual) and tile (0: 256x256, DMA-pipelined when
 * K % 32 == 0; 1: 128x128; 2: 64x64; 3: register-staged 256x256; -1: heuristic).
 * Same numerics as the entry points above. */
PK_API int pk_gemm_ex(int epi, const uint16_t *A, const uint16_t *B, uint16_t *C,
                      const uint16_t *bias, const uint16_t *R, int M, int N, int K, int tile,
                      void *stream);

/* ---- configurations (tuning-cache vocabulary) ------------------------------ */

/* One kernel configuration; the fields are those of the tuning-cache schema
 * (tuning/schema.json:65-79).  num_warps counts 64-lane waves.  In a request
 * a 0 field means "any".  Meaning per op family:
 *   GEMM (matmul, fused_matmul_bias_gelu, fused_matmul_bias_residual):
 *     block_m x block_n output tile, block_k = k-tile per LDS stage,
 *     shared_memory_stages = LDS ring depth, vector_width = bf16 per global
 *     load (8, or 1 on the unaligned path), unroll = 32x32x16 MFMA k-steps
 *     per stage.  Variants: 256x256x32 DMA ring of 4 or 5 stages (8 waves),
 *     256x256x64 register-staged (8 waves), 128x128x64 and 64x64x64 (4 waves).
 *   int8 (matmul_int8, matmul_int8_gelu, matmul_int8_residual): block_n =
 *     output columns per workgroup, split over num_warps waves of 16..256
 *     columns each; block_k = rows of K one workgroup reduces (a multiple of
 *     64; K / block_k workgroups per column slice, fp32 partials summed by a
 *     second kernel); shared_memory_stages = per-wave ring depth in 64-row
 *     steps; block_m = rows of A per workgroup (16, 32 or 64); vector_width
 *     = 16 (int8 per DMA lane); unroll = 2 (16x16x32 MFMA k-steps per step).
 *   fused_kv_append_attention (D 64 or 128): the flash kernel's two tile
 *     shapes -- block_m queries x block_n keys per step, 128 x 64 or 64 x 128
 *     (block_k = D, num_warps = 8 waves, vector_width = 8, unroll = D / 16
 *     MFMA k-steps per product, shared_memory_stages = slots of the K ring
 *     and of the V ring); other D: the generic kernel's one configuration.
 *   fused_residual_rmsnorm, fused_softmax_mask (shape rows, cols, 0):
 *     block_m = rows per workgroup (4: one wave per row; 1: one row per
 *     workgroup of num_warps = 4, 8 or 16 waves), block_n = cols, unroll =
 *     16-byte vectors per lane, vector_width 8 (1: the generic kernel for
 *     any cols), block_k 0, shared_memory_stages 1; long rows list two
 *     layouts (4 and 8 waves up to 16384 columns, 16 and 8 up to 65536;
 *     pk_fused_*_config runs either).
 *   fused_rmsnorm_matmul: one fixed configuration per shape that describes
 *     the kernel the entry point runs (see pk_op_configs). */
typedef struct pk_config {
  int block_m, block_n, block_k, num_warps, vector_width, unroll, shared_memory_stages;
} pk_config;

/* Every configuration the kernels implement for `op` at shape (M, N, K) --
 * the shape key of the op as the runtime defines it (GEMM-like ops: M, N, K;
 * row-wise ops: rows, cols, 0; fused_kv_append_attention: S_q, S_kv, D).
 * Writes min(total, cap) configurations to `out` (may be NULL when cap is 0)
 * and returns the total (0 for a shape no variant takes), or
 * PK_ERR_INVALID_ARG for an unknown op.  No device is needed. */
PK_API int pk_op_configs(const char *op, long long M, long long N, long long K, pk_config *out, int cap);
/* The configuration the op's plain entry point chooses for 16-byte aligned
 * operands (PK_ERR_UNSUPPORTED when it takes a generic fallback kernel). */
PK_API int pk_op_default_config(const char *op, long long M, long long N, long long K, pk_config *out);

/* The configuration launch_matmul_int8 would use for this shape (returns
 * PK_ERR_UNSUPPORTED when the shape takes the generic kernel). */
PK_API int pk_int8_default_config(int M, int N, int K, pk_config *out);

/* Tuning/test hook: int8 matmul with an explicit epilogue (0 none, 1 GELU,
 * 2 residual add of R [M,N]) and configuration (NULL = built-in choice).
 * Unsupported configurations return PK_ERR_UNSUPPORTED.  `workspace` (may be
 * NULL: library-owned) holds the split partials. */
PK_API int pk_matmul_int8_ex(int epi, const uint16_t *A, const int8_t *Wq, const float *scale,
                             uint16_t *C, const uint16_t *R, int M, int N, int K,
                             const pk_config *cfg, void *workspace, size_t workspace_bytes,
                             void *stream);

/* GEMM with an explicit epilogue (as pk_gemm_ex) and configuration (NULL =
 * built-in choice).  A configuration no variant matches, or one that needs
 * 16-byte aligned operands they do not have, returns PK_ERR_UNSUPPORTED. */
PK_API int pk_gemm_config_ex(int epi, const uint16_t *A, const uint16_t *B, uint16_t *C,
                             const uint16_t *bias, const uint16_t *R, int M, int N, int K,
                             const pk_config *cfg, void *stream);

/* launch_fused_kv_append_attention with an explicit configuration (one of
 * pk_op_configs("fused_kv_append_attention", S_q, S_cache + S_q, D); NULL =
 * built-in choice).  A flash configuration the operands do not allow
 * (alignment, scale <= 0, S_cache not a multiple of block_n) returns
 * PK_ERR_UNSUPPORTED; anything else not in the list PK_ERR_INVALID_ARG. */
PK_API int pk_fused_kv_append_attention_config(const uint16_t *Q, uint16_t *Kc, uint16_t *Vc, const uint16_t *Kn,
                                               const uint16_t *Vn, uint16_t *O, int B, int H, int S_q,
                                               int S_cache, int D, int cache_capacity, float scale, int causal,
                                               const pk_config *cfg, void *stream);

/* launch_fused_residual_rmsnorm / launch_fused_softmax_mask with an explicit
 * configuration (one of pk_op_configs("fused_residual_rmsnorm" or
 * "fused_softmax_mask", rows, cols, 0); NULL = built-in choice), so the
 * autotuner can time each row kernel variant (waves per row, vectors per
 * lane).  A configuration not in the list returns PK_ERR_INVALID_ARG; a
 * vector configuration (vector_width 8) with operands that are not 16-byte
 * aligned returns PK_ERR_UNSUPPORTED. */
PK_API int pk_fused_residual_rmsnorm_config(const uint16_t *x, const uint16_t *r, const uint16_t *gamma,
                                            uint16_t *out, int rows, int cols, float eps, const pk_config *cfg,
                                            void *stream);
PK_API int pk_fused_softmax_mask_config(const float *logits, const uint16_t *mask, uint16_t *out, int rows,
                                        int cols, const pk_config *cfg, void *stream);

/* Negative launch probe: launches a trivial kernel with 2048 threads per
 * workgroup (twice the limit) and stores the hipError_t of the launch and of
 * the following synchronisation.  PK_OK when the invalid launch was caught
 * (message in pk_last_error()), PK_ERR_LAUNCH if it was accepted.
 * Mirrors the `neg` mode of lib/Runtime/hip_run_main.cpp:278-309. */
PK_API int pk_probe_invalid_launch(int *launch_status, int *sync_status);

/* Launch-floor probe: an empty kernel (no memory access) with `blocks`
 * workgroups of `threads` threads and `lds_bytes` of dynamic LDS on `stream`,
 * so a benchmark can time the fixed cost of a launch of a latency-bound
 * kernel's geometry beside it.  No reference counterpart (a measurement aid
 * like benchmarks/bench_hip.cpp's timing loop). */
PK_API int pk_probe_empty_launch(int blocks, int threads, int lds_bytes, void *stream);

/* ---- code-object support ----------------------------------------------------- */
/* What a host needs to launch the emitted code objects: the device GELU table
 * of the current device (built on first use) and the library-owned workspace
 * of (current device, stream): a buffer of at least `bytes` for launches on
 * `stream` (hipStream_t; NULL = the null stream), grown on demand without a
 * device synchronisation, kept until pk_release_workspace(stream) or the end
 * of the process.  Each stream has its own buffer (hipStreamPerThread one per
 * host thread), so launches on different streams never share scratch; threads
 * that feed ONE stream must serialise their launch sequences themselves (the
 * library's own entry points hold the slot's lock while they enqueue). */
PK_API int pk_gelu_table(const uint16_t **table);
PK_API int pk_library_workspace(size_t bytes, void *stream, void **ptr);

/* Frees the library-owned workspace of (current device, stream) -- the
 * buffer the split-K / split-KV / long-row RMSNorm->MatMul paths and
 * pk_library_workspace use, and the smaller buffers it outgrew -- after
 * hipStreamSynchronize(stream), so no queued kernel still reads it.  Call it
 * before destroying a stream the library has run on (a new stream can reuse
 * the old handle value) or to return the memory; the next call on the stream
 * allocates again.  With hipStreamPerThread it frees the calling thread's
 * buffer.  PK_OK if the stream has none.  No reference counterpart (its
 * launchers own no memory, kernels/template/kernel_common.h). */
PK_API int pk_release_workspace(void *stream);

/* ---- naive device goldens (the autotuner's correctness gate) --------------- */
/* Straightforward one-thread-per-output kernels that restate the reference
 * semantics in their own sequential order (fp32 multiply then add, no
 * contraction; per-stage bf16 rounding; GELU with a double-precision erf).
 * Slow by design; asynchronous on `stream`. */
/* epi as pk_gemm_ex (0 none, 1 bias+GELU, 2 bias+residual, 3 residual). */
PK_API int pk_naive_matmul(int epi, const uint16_t *A, const uint16_t *B, uint16_t *C, const uint16_t *bias,
                           const uint16_t *R, int M, int N, int K, void *stream);
/* epi as pk_matmul_int8_ex (0 none, 1 GELU, 2 residual). */
PK_API int pk_naive_matmul_int8(int epi, const uint16_t *A, const int8_t *Wq, const float *scale, uint16_t *C,
                                const uint16_t *R, int M, int N, int K, void *stream);
/* out = rmsnorm(r ? bf16(x + r) : x, gamma, eps); r and gamma may be NULL. */
PK_API int pk_naive_rmsnorm(const uint16_t *x, const uint16_t *r, const uint16_t *gamma, uint16_t *out,
                            int rows, int cols, float eps, void *stream);
/* out = softmax(bf16(bf16(logits) + mask)). */
PK_API int pk_naive_softmax_mask(const float *logits, const uint16_t *mask, uint16_t *out, int rows, int cols,
                                 void *stream);
/* O [BH,S_q,D] over K/V rows [BH, kv_stride rows, D] (the first S_kv used). */
PK_API int pk_naive_attention(const uint16_t *Q, const uint16_t *K, const uint16_t *V, uint16_t *O, int BH,
                              int S_q, int S_kv, int kv_stride, int D, float scale, int causal, void *stream);
/* Parity metrics of got vs want (bf16, n elements) in float64: out[0] cosine,
 * out[1] max_rel_err (eps 1e-6), out[2] pcc, out[3] bit-exact fraction.
 * Definitions of tests/golden/metrics.py:20-77.  Synchronous on `stream`;
 * allocates a small device buffer. */
PK_API int pk_compare_bf16(const uint16_t *got, const uint16_t *want, long long n, double out[4], void *stream);

/* Error-model gate of the autotuner for GEMM-class outputs: *bad (host) =
 * number of outputs of `got` that are NOT the reference epilogue applied to
 * some fp32 accumulation of the same products, i.e. outside the values the
 * epilogue takes over accumulators t in S +- delta, S the exact (fp64) sum,
 * delta = (K 2^-23 + operand_ulps 2^-8) sum|p| for bf16 operands (operand_ulps
 * admits that many bf16 ulps of difference in each A element, as a fused
 * RMSNorm prologue may round a normalised activation to the neighbouring
 * bf16), (K + 2) 2^-23 sum|p| for int8 weights (the reference's per-element
 * dequantisation rounds twice per product).  Any summation order passes; a
 * wrong index, sign, dropped term or dropped bias does not.  epi as
 * pk_naive_matmul / pk_naive_matmul_int8.  Synchronous on `stream`; allocates
 * a small device buffer.  Not derived from the reference (which gates fused
 * ops on cosine / pcc only, tools/polykernel-bench/bench.py:297-306). */
PK_API int pk_gate_matmul(int epi, const uint16_t *A, const uint16_t *B, const uint16_t *bias, const uint16_t *R,
                          const uint16_t *got, int M, int N, int K, double operand_ulps, unsigned long long *bad,
                          void *stream);
PK_API int pk_gate_matmul_int8(int epi, const uint16_t *A, const int8_t *Wq, const float *scale,
                               const uint16_t *R, const uint16_t *got, int M, int N, int K,
                               unsigned long long *bad, void *stream);

/* ---- synthetic inputs (host, deterministic, OpenMP) -------------------- */

/* out[i] = bf16 RNE of float(mean + std * z_i), z_i standard normal from the
 * counter-based generator (SplitMix64 -> Box-Muller in double) at (seed,
 * stream_id, i).  Identical output for any thread count. */
PK_API void pk_synth_normal_bf16(uint64_t seed, uint64_t stream_id, double mean, double std, uint16_t *out,
                          int64_t n);
/* Same draws, kept as fp32. */
PK_API void pk_synth_normal_f32(uint64_t seed, uint64_t stream_id, double mean, double std, float *out,
                         int64_t n);
/* Additive bf16 mask: -inf (0xFF80) with probability p, else +0. */
PK_API void pk_synth_mask_bf16(uint64_t seed, uint64_t stream_id, double p, uint16_t *out, int64_t n);

#ifdef __cplusplus
}
#endif

#endif /* POLYKERNEL_AMD_H */
