// gemm.hip -- bf16 MFMA GEMM for gfx950 with fused epilogues.
//
// C[M,N] = A[M,K] @ B[K,N] with A K-contiguous and B N-contiguous (the
// reference layouts, kernels/cpu/cpu_reference.cpp:64-78), fp32 accumulation on
// v_mfma_f32_32x32x16_bf16.  Per workgroup a BM x BN tile; WM x WN waves, each
// owning a (BM/WM) x (BN/WN) sub-tile of 32x32 MFMA blocks.  A and B k-tiles of
// 64 are staged through LDS, double-buffered with one barrier per k-tile:
//   - A rows (128 B) are stored with 16-byte chunks XOR-swizzled by
//     (row >> 1) & 7, read as one ds_read_b128 per MFMA A-operand;
//   - B rows keep the global N-contiguous order (16-byte chunks swizzled by
//     k), and the MFMA B-operand (8 consecutive k of one column) is assembled
//     by two ds_read_b64_tr_b16 transpose reads, so no pre-packed weights and
//     no register transposes are needed.
// Workgroups are remapped so each XCD gets a contiguous band of tiles, rastered
// in groups of tile-rows for L2 reuse.
//
// Epilogues reproduce the golden per-stage bf16 rounding
// (tests/golden/golden.py:48-66, kernels/cpu/cpu_reference.cpp:92-105):
//   EPI_NONE        c = bf16(acc)
//   EPI_BIAS_GELU   c = gelu(bf16(bf16(acc) + bias[n]))      (exact GELU, gelu_bits)
//   EPI_BIAS_RESID  c = bf16(bf16(bf16(acc) + bias[n]) + R[m,n])
//   EPI_RESID       c = bf16(bf16(acc) + R[m,n])
#include <type_traits>

#include "gemm_kernels.hpp"

namespace pk {


namespace {

using namespace gk;

// The kernels, as the library launches them (bodies in gemm_kernels.hpp).
template <int BM, int BN, int WM, int WN, int EPI, bool ALIGNED>
__global__ __launch_bounds__(WM *WN * 64) void gemm_kernel(GemmArgs g) {
  gemm_reg_body<BM, BN, WM, WN, EPI, ALIGNED>(g);
}

template <int EPI, int STAGES, int W = G2_WAVES, int WNN = G2_WAVES_N>
__global__ __launch_bounds__(W * 64, 1) void gemm_dma_kernel(GemmArgs g) {
  gemm_dma_body<EPI, STAGES, W, WNN>(g);
}

template <int BM, int BN, int WM, int WN, int EPI>
int launch_tile(const GemmArgs &g, bool aligned, hipStream_t st) {
  const int tiles = ((g.M + BM - 1) / BM) * ((g.N + BN - 1) / BN);
  if (aligned)
    gemm_kernel<BM, BN, WM, WN, EPI, true><<<tiles, WM * WN * 64, 0, st>>>(g);
  else
    gemm_kernel<BM, BN, WM, WN, EPI, false><<<tiles, WM * WN * 64, 0, st>>>(g);
  PK_LAUNCH_CHECK("gemm_kernel");
  return PK_OK;
}

// The kernels map blockIdx.x to (tile row, tile column) and round M, N and K
// up to whole tiles in 32-bit arithmetic: each stays 1023 below INT32_MAX,
// and a grid of the smallest tile (bm x bn) within INT32_MAX workgroups.
int tile_grid_ok(int M, int N, int K, int bm, int bn, const char *name) {
  if (M > INT32_MAX - 1023 || N > INT32_MAX - 1023 || K > INT32_MAX - 1023) {
    set_error("%s: M=%d, N=%d or K=%d is within 1023 of INT32_MAX", name, M, N, K);
    return PK_ERR_UNSUPPORTED;
  }
  if ((((int64_t)M + bm - 1) / bm) * (((int64_t)N + bn - 1) / bn) <= INT32_MAX) return PK_OK;
  set_error("%s: M=%d x N=%d needs more than %d workgroups", name, M, N, INT32_MAX);
  return PK_ERR_UNSUPPORTED;
}

// Whether tile 0 runs the direct-to-LDS 256x256 kernel for these operands
// (otherwise the register-staged one).
bool gemm_dma_fits(const GemmArgs &g) {
  const bool aligned = (g.K % 8 == 0) && (g.N % 8 == 0) && aligned16(g.A) && aligned16(g.B);
  const bool offsets32 = (size_t)g.K * g.N * 2 < (size_t(1) << 31) &&
                         (size_t)G2_BM * g.K * 2 < (size_t(1) << 31);
  const bool ep_aligned = aligned16(g.C) && (!g.R || aligned16(g.R)) && (!g.bias || aligned16(g.bias));
  return aligned && ep_aligned && offsets32 && g.K % G2_BK == 0 && g.N >= 8;
}

template <int EPI>
int gemm_dispatch(const GemmArgs &g, int tile, hipStream_t st) {
  const bool aligned = (g.K % 8 == 0) && (g.N % 8 == 0) && aligned16(g.A) && aligned16(g.B);
  if (tile == 0 && gemm_dma_fits(g)) {
    const int tiles = ((g.M + G2_BM - 1) / G2_BM) * ((g.N + G2_BN - 1) / G2_BN);
    gemm_dma_kernel<EPI, 5><<<tiles, G2_THREADS, 0, st>>>(g);
    PK_LAUNCH_CHECK("gemm_dma_kernel");
    return PK_OK;
  }
  if (tile == 3) tile = 0;  // the 8-wave register-staged 256x256 kernel
  switch (tile) {
    case 0: return launch_tile<256, 256, 2, 4, EPI>(g, aligned, st);
    case 1: return launch_tile<128, 128, 2, 2, EPI>(g, aligned, st);
    default: return launch_tile<64, 64, 2, 2, EPI>(g, aligned, st);
  }
}

// ---- configurations in the tuning-cache vocabulary ------------------------
// Variants, in order of preference: the DMA ring at 5 and 4 stages, then the
// register-staged kernels.  vector_width 8 needs K % 8 == 0, N % 8 == 0 and
// 16-byte aligned operands; 1 is the element-wise load path.
enum GemmVariant { GV_DMA5, GV_DMA4, GV_REG256, GV_REG128, GV_REG64, GV_COUNT };

pk_config gemm_variant_config(int v, int vw) {
  switch (v) {
    case GV_DMA5: return pk_config{G2_BM, G2_BN, G2_BK, G2_THREADS / 64, 8, G2_BK / 16, 5};
    case GV_DMA4: return pk_config{G2_BM, G2_BN, G2_BK, G2_THREADS / 64, 8, G2_BK / 16, 4};
    case GV_REG256: return pk_config{256, 256, BK, 8, vw, BK / 16, 2};
    case GV_REG128: return pk_config{128, 128, BK, 4, vw, BK / 16, 2};
    default: return pk_config{64, 64, BK, 4, vw, BK / 16, 2};
  }
}

bool gemm_dma_shape_ok(int N, int K) {
  return K % G2_BK == 0 && N % 8 == 0 && N >= 8 && (size_t)K * N * 2 < (size_t(1) << 31) &&
         (size_t)G2_BM * K * 2 < (size_t(1) << 31);
}

bool cfg_matches(const pk_config &req, const pk_config &c) {
  return (!req.block_m || req.block_m == c.block_m) && (!req.block_n || req.block_n == c.block_n) &&
         (!req.block_k || req.block_k == c.block_k) && (!req.num_warps || req.num_warps == c.num_warps) &&
         (!req.vector_width || req.vector_width == c.vector_width) && (!req.unroll || req.unroll == c.unroll) &&
         (!req.shared_memory_stages || req.shared_memory_stages == c.shared_memory_stages);
}

template <int EPI>
int gemm_launch_variant(const GemmArgs &g, int v, bool vec, hipStream_t st) {
  switch (v) {
    case GV_DMA5:
      gemm_dma_kernel<EPI, 5><<<((g.M + G2_BM - 1) / G2_BM) * ((g.N + G2_BN - 1) / G2_BN), G2_THREADS, 0, st>>>(g);
      PK_LAUNCH_CHECK("gemm_dma_kernel");
      return PK_OK;
    case GV_DMA4:
      gemm_dma_kernel<EPI, 4><<<((g.M + G2_BM - 1) / G2_BM) * ((g.N + G2_BN - 1) / G2_BN), G2_THREADS, 0, st>>>(g);
      PK_LAUNCH_CHECK("gemm_dma_kernel");
      return PK_OK;
    case GV_REG256: return launch_tile<256, 256, 2, 4, EPI>(g, vec, st);
    case GV_REG128: return launch_tile<128, 128, 2, 2, EPI>(g, vec, st);
    default: return launch_tile<64, 64, 2, 2, EPI>(g, vec, st);
  }
}

// Largest tile that still gives at least ~one workgroup per CU.
// With the direct-to-LDS kernel (`dma`), 256x256 from 72 tiles up: even one
// round that leaves most CUs idle beats the 128x128 kernel's rounds (K 4096:
// [1280, 4096] 80 tiles 69.5 against 73.0 us, [2048, 4096] 128 tiles 72.1
// against 84.6, [3072, 3072] 144 tiles 73.4 against 137.0, [2048, 6144] 192
// tiles 87.4 against 141.4), while at 64 tiles one full round of 128x128
// tiles wins ([1024, 4096] 59.4 against 68.9 us).  The register-staged
// 256x256 kernel keeps the 200-tile threshold; 64x64 below 200 128x128
// tiles ([512, 4096] 41.4 against 57.4 us for 128x128).
int pick_tile(int M, int N, bool dma) {
  const long t256 = (((long)M + 255) / 256) * (((long)N + 255) / 256);
  const long t128 = (((long)M + 127) / 128) * (((long)N + 127) / 128);
  if (t256 >= (dma ? 72 : 200)) return 0;
  if (t128 >= 200) return 1;
  return 2;
}

}  // namespace

int gemm_configs(int M, int N, int K, pk_config *out, int cap) {
  if (M <= 0 || N <= 0 || K <= 0) return 0;
  const int vw = (K % 8 == 0 && N % 8 == 0) ? 8 : 1;
  int n = 0;
  for (int v = 0; v < GV_COUNT; ++v) {
    if ((v == GV_DMA5 || v == GV_DMA4) && !gemm_dma_shape_ok(N, K)) continue;
    if (out && n < cap) out[n] = gemm_variant_config(v, vw);
    ++n;
    if (vw == 8 && v >= GV_REG256) {  // the element-wise load path is always there too
      if (out && n < cap) out[n] = gemm_variant_config(v, 1);
      ++n;
    }
  }
  return n;
}

// What gemm_run picks for 16-byte aligned operands.
bool gemm_default(int M, int N, int K, pk_config *out) {
  if (M <= 0 || N <= 0 || K <= 0) return false;
  const int vw = (K % 8 == 0 && N % 8 == 0) ? 8 : 1;
  const bool dma = vw == 8 && gemm_dma_shape_ok(N, K);
  const int tile = pick_tile(M, N, dma);
  int v = tile == 0 ? GV_REG256 : tile == 1 ? GV_REG128 : GV_REG64;
  if (tile == 0 && dma) v = GV_DMA5;
  *out = gemm_variant_config(v, vw);
  return true;
}

int gemm_run_config(int epi, const uint16_t *A, const uint16_t *B, uint16_t *C, const uint16_t *bias,
                    const uint16_t *R, int M, int N, int K, const pk_config &req, hipStream_t st) {
  if (int rc = tile_grid_ok(M, N, K, 64, 64, "matmul")) return rc;
  GemmArgs g{A, B, C, bias, R, nullptr, M, N, K};
  const bool shape_vec = (K % 8 == 0) && (N % 8 == 0);
  const bool ptr_vec = aligned16(A) && aligned16(B);
  const bool ep_aligned = aligned16(C) && (!R || aligned16(R)) && (!bias || aligned16(bias));
  int chosen = -1;
  bool vec = false;
  for (int v = 0; v < GV_COUNT && chosen < 0; ++v) {
    if ((v == GV_DMA5 || v == GV_DMA4) && !(gemm_dma_shape_ok(N, K) && ptr_vec && ep_aligned)) continue;
    for (int vw : {8, 1}) {
      if (vw == 8 && !(shape_vec && ptr_vec)) continue;
      if (vw == 1 && (v == GV_DMA5 || v == GV_DMA4)) continue;
      if (cfg_matches(req, gemm_variant_config(v, vw))) {
        chosen = v;
        vec = vw == 8;
        break;
      }
    }
  }
  if (chosen < 0) {
    set_error("gemm: configuration {block_m %d, block_n %d, block_k %d, num_warps %d, vector_width %d, "
              "unroll %d, stages %d} not available for M=%d N=%d K=%d with these operand alignments",
              req.block_m, req.block_n, req.block_k, req.num_warps, req.vector_width, req.unroll,
              req.shared_memory_stages, M, N, K);
    return PK_ERR_UNSUPPORTED;
  }
  if (epi == EPI_BIAS_GELU) {
    int rc = gelu_table(&g.gelu_tab);
    if (rc) return rc;
  }
  switch (epi) {
    case EPI_NONE: return gemm_launch_variant<EPI_NONE>(g, chosen, vec, st);
    case EPI_BIAS_GELU: return gemm_launch_variant<EPI_BIAS_GELU>(g, chosen, vec, st);
    case EPI_BIAS_RESID: return gemm_launch_variant<EPI_BIAS_RESID>(g, chosen, vec, st);
    default: return gemm_launch_variant<EPI_RESID>(g, chosen, vec, st);
  }
}

int gemm_run(int epi, const uint16_t *A, const uint16_t *B, uint16_t *C, const uint16_t *bias,
             const uint16_t *R, int M, int N, int K, hipStream_t st, int tile = -1) {
  if (int rc = tile_grid_ok(M, N, K, 64, 64, "matmul")) return rc;
  GemmArgs g{A, B, C, bias, R, nullptr, M, N, K};
  if (epi == EPI_BIAS_GELU) {
    int rc = gelu_table(&g.gelu_tab);
    if (rc) return rc;
  }
  if (tile < 0) tile = pick_tile(M, N, gemm_dma_fits(g));
  switch (epi) {
    case EPI_NONE: return gemm_dispatch<EPI_NONE>(g, tile, st);
    case EPI_BIAS_GELU: return gemm_dispatch<EPI_BIAS_GELU>(g, tile, st);
    case EPI_BIAS_RESID: return gemm_dispatch<EPI_BIAS_RESID>(g, tile, st);
    default: return gemm_dispatch<EPI_RESID>(g, tile, st);
  }
}

// The RMSNorm -> MatMul panel kernel (body in gemm_kernels.hpp).
__global__ __launch_bounds__(RQ_THREADS) void rmsnorm_panel_gemm_fast_kernel(PanelArgs a) {
  rmsnorm_panel_fast_body(a);
}

int rmsnorm_launch(const uint16_t *x, const uint16_t *w, uint16_t *y, int rows, int cols,
                   float eps, hipStream_t st);

// The whole-K panel kernel (x panel and W slice in LDS, 32 x 64 tiles) when K
// <= 832 and its grid is one round of at most 256 tiles: a latency kernel
// that reloads W for every 32 rows, so past one round RMSNorm into workspace
// and the GEMM win (K 768: M 128 8.4 against 13.2 us; M 192 14.9 against 13.3;
// M 1024 56.5 against 21.7; [4096, 4096] 215.8 against 36.5 us).  The
// double-buffered panel kernel (2 waves, 64-deep k-tiles, K <= 1536) lost at
// every measured shape (M 16-128, N 4096, K 1024: 25.9-34.9 against 14.0-15.2
// us; [4096, 4096, 1024] 1152.6 against 43.0 us) and was removed.
bool fast_panel_fits(int M, int N, int K) {
  const long tiles = (((long)M + RQ_BM - 1) / RQ_BM) * (((long)N + RQ_BN - 1) / RQ_BN);
  return K <= RQ_MAX_K && tiles <= 256 && (size_t)K * N * 2 < (size_t(1) << 31);
}

// The kernel fused_rmsnorm_matmul runs for aligned operands, as a config: the
// whole-K panel kernel where fast_panel_fits, otherwise row normalisation into
// workspace followed by the GEMM's own choice.
bool rmsnorm_matmul_config(int M, int N, int K, pk_config *out) {
  if (M <= 0 || N <= 0 || K <= 0) return false;
  const bool panel_ok = (K % BK == 0) && (N % 8 == 0);
  if (panel_ok && fast_panel_fits(M, N, K)) {
    *out = pk_config{RQ_BM, RQ_BN, K, RQ_THREADS / 64, 8, K / 16, 1};
    return true;
  }
  return gemm_default(M, N, K, out);
}

int fused_rmsnorm_matmul(const uint16_t *x, const uint16_t *gamma, const uint16_t *W, uint16_t *out,
                         int M, int N, int K, float eps, hipStream_t st, const char *name) {
  PK_CHECK_ARG(x && W && out, "%s: null tensor pointer", name);
  PK_CHECK_ARG(M >= 0 && N >= 0 && K > 0, "%s: invalid shape M=%d N=%d K=%d", name, M, N, K);
  if (M == 0 || N == 0) return PK_OK;
  if (int rc = tile_grid_ok(M, N, K, RQ_BM, RQ_BN, name)) return rc;
  const bool panel_ok = (K % BK == 0) && (N % 8 == 0) && aligned16(x) &&
                        aligned16(W) && (!gamma || aligned16(gamma));
  if (panel_ok && fast_panel_fits(M, N, K) && aligned16(out)) {
    const int tiles = ((M + RQ_BM - 1) / RQ_BM) * ((N + RQ_BN - 1) / RQ_BN);
    const size_t lds = pk_panel_lds_bytes(K);
    rmsnorm_panel_gemm_fast_kernel<<<tiles, RQ_THREADS, lds, st>>>(
        PanelArgs{x, gamma, W, out, M, N, K, 1.0f / (float)K, eps});
    PK_LAUNCH_CHECK(name);
    return PK_OK;
  }
  // Otherwise: normalise once into library workspace, then the plain GEMM.
  WorkspaceLease lease;  // held until the GEMM that reads the panel is queued
  int rc = library_workspace((size_t)M * K * 2, st, lease);
  if (rc) return rc;
  uint16_t *a = static_cast<uint16_t *>(lease.ptr);
  rc = rmsnorm_launch(x, gamma, a, M, K, eps, st);
  if (rc) return rc;
  return gemm_run(EPI_NONE, a, W, out, nullptr, nullptr, M, N, K, st);
}

}  // namespace pk

using namespace pk;

extern "C" {

int launch_matmul(const uint16_t *A, const uint16_t *B, uint16_t *C, int M, int N, int K,
                  void *stream) {
  PK_CHECK_ARG(A && B && C, "launch_matmul: null tensor pointer");
  PK_CHECK_ARG(M >= 0 && N >= 0 && K >= 0, "launch_matmul: invalid shape");
  if (M == 0 || N == 0) return PK_OK;
  PK_CHECK_ARG(K > 0, "launch_matmul: K must be positive");
  return gemm_run(EPI_NONE, A, B, C, nullptr, nullptr, M, N, K, (hipStream_t)stream);
}

int launch_fused_matmul_bias_gelu(const uint16_t *a, const uint16_t *b, const uint16_t *bias,
                                  uint16_t *output, int M, int N, int K, void *stream) {
  PK_CHECK_ARG(a && b && bias && output, "launch_fused_matmul_bias_gelu: null tensor pointer");
  PK_CHECK_ARG(M >= 0 && N >= 0 && K > 0, "launch_fused_matmul_bias_gelu: invalid shape");
  if (M == 0 || N == 0) return PK_OK;
  return gemm_run(EPI_BIAS_GELU, a, b, output, bias, nullptr, M, N, K, (hipStream_t)stream);
}

int launch_fused_matmul_bias_residual(const uint16_t *a, const uint16_t *b, const uint16_t *bias,
                                      const uint16_t *residual, uint16_t *out, int M, int N, int K,
                                      void *stream) {
  PK_CHECK_ARG(a && b && residual && out, "launch_fused_matmul_bias_residual: null tensor pointer");
  PK_CHECK_ARG(M >= 0 && N >= 0 && K > 0, "launch_fused_matmul_bias_residual: invalid shape");
  if (M == 0 || N == 0) return PK_OK;
  return gemm_run(bias ? EPI_BIAS_RESID : EPI_RESID, a, b, out, bias, residual, M, N, K,
                  (hipStream_t)stream);
}

int launch_fused_rmsnorm_matmul(const uint16_t *input, const uint16_t *weight, uint16_t *output,
                                int M, int N, int K, float eps, void *stream) {
  return fused_rmsnorm_matmul(input, nullptr, weight, output, M, N, K, eps, (hipStream_t)stream,
                              "launch_fused_rmsnorm_matmul");
}

int launch_fused_rmsnorm_matmul_gamma(const uint16_t *x, const uint16_t *gamma, const uint16_t *W,
                                      uint16_t *out, int M, int N, int K, float eps, void *stream) {
  return fused_rmsnorm_matmul(x, gamma, W, out, M, N, K, eps, (hipStream_t)stream,
                              "launch_fused_rmsnorm_matmul_gamma");
}

size_t pk_mlp_block_workspace_size(int M, int d, int F) {
  if (M <= 0 || d <= 0 || F <= 0) return 0;  // no launch takes a workspace
  auto up = [](size_t v) { return (v + 255) & ~size_t(255); };
  return up((size_t)M * d * 2) + up((size_t)M * F * 2);
}

int launch_mlp_block(const uint16_t *x, const uint16_t *gamma, const uint16_t *W1,
                     const uint16_t *b1, const uint16_t *W2, const uint16_t *b2, uint16_t *out,
                     int M, int d, int F, float eps, void *workspace, size_t workspace_bytes,
                     void *stream) {
  PK_CHECK_ARG(x && W1 && b1 && W2 && b2 && out, "launch_mlp_block: null tensor pointer");
  PK_CHECK_ARG(M >= 0 && d > 0 && F > 0, "launch_mlp_block: invalid shape");
  if (M == 0) return PK_OK;
  if (int rc = tile_grid_ok(M, std::max(d, F), std::max(d, F), 64, 64, "launch_mlp_block")) return rc;  // before any launch
  const size_t need = pk_mlp_block_workspace_size(M, d, F);
  if (!workspace || workspace_bytes < need) {
    set_error("launch_mlp_block: workspace of %zu bytes required, got %zu", need, workspace_bytes);
    return PK_ERR_WORKSPACE;
  }
  hipStream_t st = (hipStream_t)stream;
  uint16_t *a = static_cast<uint16_t *>(workspace);
  uint16_t *h = a + (((size_t)M * d * 2 + 255) & ~size_t(255)) / 2;
  int rc = rmsnorm_launch(x, gamma, a, M, d, eps, st);
  if (rc) return rc;
  rc = gemm_run(EPI_BIAS_GELU, a, W1, h, b1, nullptr, M, F, d, st);
  if (rc) return rc;
  return gemm_run(EPI_BIAS_RESID, h, W2, out, b2, x, M, d, F, st);
}

// Test/tuning hook: run one GEMM epilogue variant with an explicit tile choice
// (0: 256x256 -- the DMA-pipelined kernel when K % 32 == 0 and the operands
// are aligned, 1: 128x128, 2: 64x64, 3: the register-staged 256x256 kernel;
// -1: heuristic).
int pk_gemm_config_ex(int epi, const uint16_t *A, const uint16_t *B, uint16_t *C, const uint16_t *bias,
                      const uint16_t *R, int M, int N, int K, const pk_config *cfg, void *stream) {
  PK_CHECK_ARG(A && B && C, "pk_gemm_config_ex: null tensor pointer");
  PK_CHECK_ARG(M > 0 && N > 0 && K > 0, "pk_gemm_config_ex: invalid shape");
  PK_CHECK_ARG(epi >= 0 && epi <= 3, "pk_gemm_config_ex: epilogue %d not in 0..3", epi);
  PK_CHECK_ARG((epi != EPI_BIAS_GELU || bias) && (epi < EPI_BIAS_RESID || R),
               "pk_gemm_config_ex: epilogue %d needs its bias/residual operand", epi);
  if (!cfg) return gemm_run(epi, A, B, C, bias, R, M, N, K, (hipStream_t)stream);
  return gemm_run_config(epi, A, B, C, bias, R, M, N, K, *cfg, (hipStream_t)stream);
}

int pk_gemm_ex(int epi, const uint16_t *A, const uint16_t *B, uint16_t *C, const uint16_t *bias,
               const uint16_t *R, int M, int N, int K, int tile, void *stream) {
  PK_CHECK_ARG(A && B && C, "pk_gemm_ex: null tensor pointer");
  PK_CHECK_ARG(M > 0 && N > 0 && K > 0, "pk_gemm_ex: invalid shape");
  PK_CHECK_ARG(epi >= 0 && epi <= 3 && tile >= -1 && tile <= 3, "pk_gemm_ex: bad epi/tile");
  return gemm_run(epi, A, B, C, bias, R, M, N, K, (hipStream_t)stream, tile);
}

}  // extern "C"
