// launchers.cpp -- the LaunchFn of every built-in op: the serving half of
// Runtime::Run (detect -> select -> serve).
//
// Each launcher receives the selected cache entry and the op's argument
// block.  It refuses an argument block whose dimensions are not the entry's
// shape and an entry whose config is not one the kernels implement for that
// shape (a hand-edited or foreign cache entry is an error, never a silent
// re-tune), then launches through the C-ABI with the entry's config.  The
// reference's LaunchFn contract is lib/Runtime/Runtime.h:47-48.
#include <algorithm>

#include "../../../include/polykernel_amd_runtime.hpp"

namespace pk::runtime {

namespace {

pk_config ToPk(const Config &c) {
  return pk_config{c.block_m, c.block_n, c.block_k, c.num_warps, c.vector_width, c.unroll, c.shared_memory_stages};
}

bool CheckEntry(const CacheEntry &e, std::int64_t m, std::int64_t n, std::int64_t k, std::string &error) {
  if (e.shape.m != m || e.shape.n != n || e.shape.k != k) {
    error = "argument block shape M=" + std::to_string(m) + ",N=" + std::to_string(n) + ",K=" + std::to_string(k) +
            " does not match the selected entry " + FormatKey(e.gpu, e.op, e.shape);
    return false;
  }
  const std::vector<Config> cands = autotune::ConfigSpace::Candidates(e.op, e.shape);
  if (std::find(cands.begin(), cands.end(), e.best) == cands.end()) {
    error = "cached config {" + autotune::ToString(e.best) + "} for " + FormatKey(e.gpu, e.op, e.shape) +
            " is not one the gfx950 kernels implement; re-run the autotuner";
    return false;
  }
  return true;
}

bool Launched(int rc, const CacheEntry &e, std::string &error) {
  if (rc == PK_OK) return true;
  error = "hip launch failed for " + FormatKey(e.gpu, e.op, e.shape) + " (status " + std::to_string(rc) +
          "): " + pk_last_error();
  return false;
}

template <typename IO>
IO *Cast(void *io, std::string &error) {
  if (io == nullptr) error = "null argument block";
  return static_cast<IO *>(io);
}

LaunchFn GemmLauncher(int epi) {
  return [epi](const CacheEntry &e, void *io, std::string &error) {
    MatmulIO *p = Cast<MatmulIO>(io, error);
    if (!p || !CheckEntry(e, p->M, p->N, p->K, error)) return false;
    const pk_config c = ToPk(e.best);
    return Launched(pk_gemm_config_ex(epi, p->A, p->B, p->C, p->bias, epi >= 2 ? p->residual : nullptr, p->M, p->N,
                                      p->K, &c, p->stream),
                    e, error);
  };
}

LaunchFn Int8Launcher(int epi) {
  return [epi](const CacheEntry &e, void *io, std::string &error) {
    MatmulInt8IO *p = Cast<MatmulInt8IO>(io, error);
    if (!p || !CheckEntry(e, p->M, p->N, p->K, error)) return false;
    const pk_config c = ToPk(e.best);
    return Launched(pk_matmul_int8_ex(epi, p->A, p->Wq, p->scale, p->C, epi == 2 ? p->residual : nullptr, p->M, p->N,
                                      p->K, &c, p->workspace, p->workspace_bytes, p->stream),
                    e, error);
  };
}

}  // namespace

void RegisterBuiltinLaunchers(Runtime &rt) {
  rt.RegisterLauncher("matmul", GemmLauncher(0));
  rt.RegisterLauncher("fused_matmul_bias_gelu", GemmLauncher(1));
  rt.RegisterLauncher("fused_matmul_bias_residual", GemmLauncher(2));
  rt.RegisterLauncher("matmul_int8", Int8Launcher(0));
  rt.RegisterLauncher("matmul_int8_gelu", Int8Launcher(1));
  rt.RegisterLauncher("matmul_int8_residual", Int8Launcher(2));
  rt.RegisterLauncher("fused_rmsnorm_matmul", [](const CacheEntry &e, void *io, std::string &error) {
    RmsnormMatmulIO *p = Cast<RmsnormMatmulIO>(io, error);
    if (!p || !CheckEntry(e, p->M, p->N, p->K, error)) return false;
    return Launched(
        launch_fused_rmsnorm_matmul_gamma(p->x, p->gamma, p->W, p->out, p->M, p->N, p->K, p->eps, p->stream), e,
        error);
  });
  rt.RegisterLauncher("fused_residual_rmsnorm", [](const CacheEntry &e, void *io, std::string &error) {
    ResidualRmsnormIO *p = Cast<ResidualRmsnormIO>(io, error);
    if (!p || !CheckEntry(e, p->rows, p->cols, 0, error)) return false;
    return Launched(
        launch_fused_residual_rmsnorm(p->x, p->r, p->gamma, p->out, p->rows, p->cols, p->eps, p->stream), e, error);
  });
  rt.RegisterLauncher("fused_softmax_mask", [](const CacheEntry &e, void *io, std::string &error) {
    SoftmaxMaskIO *p = Cast<SoftmaxMaskIO>(io, error);
    if (!p || !CheckEntry(e, p->rows, p->cols, 0, error)) return false;
    return Launched(launch_fused_softmax_mask(p->logits, p->mask, p->out, p->rows, p->cols, p->stream), e, error);
  });
  rt.RegisterLauncher("fused_kv_append_attention", [](const CacheEntry &e, void *io, std::string &error) {
    KvAppendAttentionIO *p = Cast<KvAppendAttentionIO>(io, error);
    if (!p || !CheckEntry(e, p->S_q, (std::int64_t)p->S_cache + p->S_q, p->D, error)) return false;
    return Launched(launch_fused_kv_append_attention(p->Q, p->Kc, p->Vc, p->Kn, p->Vn, p->O, p->B, p->H, p->S_q,
                                                     p->S_cache, p->D, p->cache_capacity, p->scale, p->causal,
                                                     p->stream),
                    e, error);
  });
}

}  // namespace pk::runtime
