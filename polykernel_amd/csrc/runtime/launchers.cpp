// launchers.cpp -- the LaunchFn of every built-in op: the serving half of
// Runtime::Run (detect -> select -> serve).
//
// Each launcher receives the selected cache entry and the op's argument
// block.  It refuses an argument block whose dimensions are not the entry's
// shape and an entry whose config is not one the kernels implement for that
// shape (a hand-edited or foreign cache entry is an error, never a silent
// re-tune), then launches through the C-ABI with the entry's config.  The
// reference's LaunchFn contract is lib/Runtime/Runtime.h:47-48.
#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <initializer_list>
#include <map>
#include <memory>
#include <mutex>

#include "../../../include/polykernel_amd_runtime.hpp"
#include "../attention_module.hpp"
#include "internal.hpp"
#include "../gemm_args.h"
#include "../int8_args.h"
#include "../rowwise_args.h"
#include "../workspace.hpp"

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

// Code objects loaded by the code-object launchers, keyed by path and hash.
struct ModuleTable {
  struct Loaded {
    CodeObject module;
    std::vector<void *> fns;  // the entry points asked for, in order
  };
  const KernelCache &cache;
  std::mutex mu;
  std::map<std::string, std::unique_ptr<Loaded>> loaded;

  explicit ModuleTable(const KernelCache &c) : cache(c) {}

  // The module of `bin` with the entry points `names` resolved (an object
  // serves one op, so the names are the same on every call for a binary).
  Loaded *Get(const CachedBinary &bin, std::initializer_list<const char *> names, std::string &error) {
    std::lock_guard<std::mutex> lock(mu);
    const std::string key = bin.so_path + "#" + bin.kernel_hash;
    auto it = loaded.find(key);
    if (it != loaded.end()) return it->second.get();
    auto l = std::make_unique<Loaded>();
    if (!l->module.Load(bin, error)) return nullptr;
    for (const char *n : names) {
      void *f = l->module.Function(n, error);
      if (!f) return nullptr;
      l->fns.push_back(f);
    }
    Loaded *raw = l.get();
    loaded.emplace(key, std::move(l));
    return raw;
  }
};

bool Aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

template <typename Args>
bool ModuleLaunch(void *fn, unsigned gx, unsigned gy, unsigned threads, void *stream, Args &args, const char *what,
                  std::string &error, unsigned lds_bytes = 0) {
  void *params[] = {&args};
  const hipError_t e = hipModuleLaunchKernel(static_cast<hipFunction_t>(fn), gx, gy, 1, threads, 1, 1, lds_bytes,
                                             static_cast<hipStream_t>(stream), params, nullptr);
  if (e != hipSuccess) {
    error = std::string("hip launch failed for ") + what + ": " + hipGetErrorString(e);
    (void)hipGetLastError();
    return false;
  }
  return true;
}

// Workgroups of an output tiling of [M, N] by bm x bn tiles; the kernels
// round M, N and K up to tiles and decode blockIdx.x in 32-bit arithmetic, so
// a dimension within 1023 of INT32_MAX, or more than INT32_MAX tiles, is an
// error.
bool TileGrid(int M, int N, int K, int bm, int bn, unsigned &tiles, std::string &error) {
  if (bm <= 0 || bn <= 0 || M > INT32_MAX - 1023 || N > INT32_MAX - 1023 || K > INT32_MAX - 1023) {
    error = "output tiling of " + std::to_string(M) + " x " + std::to_string(N) + " by " + std::to_string(bm) +
            " x " + std::to_string(bn) + ": tiles must be positive and M, N, K at least 1023 below INT32_MAX";
    return false;
  }
  const long long t = (((long long)M + bm - 1) / bm) * (((long long)N + bn - 1) / bn);
  if (t > INT32_MAX) {
    error = "output tiling of " + std::to_string(M) + " x " + std::to_string(N) + " by " + std::to_string(bm) +
            " x " + std::to_string(bn) + " needs more than INT32_MAX workgroups";
    return false;
  }
  tiles = (unsigned)t;
  return true;
}

// The launch geometry of an int8 config follows from its fields: column
// slices of block_n, K splits of block_k rows (64-row steps), row blocks of
// block_m; the streaming kernel and, with more than one split, the split
// reduction (as int8_run launches them).
LaunchFn CodeObjectInt8Launcher(int epi, std::shared_ptr<ModuleTable> table) {
  return [epi, table](const CacheEntry &e, void *io, std::string &error) {
    MatmulInt8IO *p = Cast<MatmulInt8IO>(io, error);
    if (!p) return false;
    // the linked path's argument check (pk_matmul_int8_ex), before any device call
    if (!p->A || !p->Wq || !p->scale || !p->C || (epi == 2 && !p->residual)) {
      error = "matmul_int8 code object: null tensor pointer";
      return false;
    }
    if (!CheckEntry(e, p->M, p->N, p->K, error)) return false;
    const std::optional<CachedBinary> bin = table->cache.GetBinary(e.gpu, e.op, e.shape);
    if (!bin) {
      error = "no code object cached for " + FormatKey(e.gpu, e.op, e.shape) +
              "; emit one (python -m polykernel_amd.emit)";
      return false;
    }
    ModuleTable::Loaded *mod = table->Get(*bin, {"pk_int8_stream", "pk_int8_reduce"}, error);
    if (!mod) return false;
    if (!Aligned16(p->A) || !Aligned16(p->Wq) || !Aligned16(p->scale) || !Aligned16(p->C) ||
        (epi == 2 && !Aligned16(p->residual))) {
      error = "code-object int8 launch needs 16-byte aligned A, Wq, scale, C and residual";
      return false;
    }
    const Config &c = e.best;
    const int ksteps = p->K / 64;
    const int split_steps = std::min(ksteps, c.block_k / 64);
    const int splits = (ksteps + split_steps - 1) / split_steps;
    const int slices = (p->N + c.block_n - 1) / c.block_n;
    const int mblocks = (p->M + c.block_m - 1) / c.block_m;
    void *ws = nullptr;
    WorkspaceLease lease;  // library scratch, held until the reduction is queued
    if (splits > 1) {
      const size_t need = (size_t)splits * p->M * p->N * sizeof(float);
      if (p->workspace) {
        if (p->workspace_bytes < need || !Aligned16(p->workspace)) {
          error = "workspace of " + std::to_string(need) + " aligned bytes required";
          return false;
        }
        ws = p->workspace;
      } else if (library_workspace(need, p->stream, lease) != PK_OK) {
        error = std::string("library workspace: ") + pk_last_error();
        return false;
      } else {
        ws = lease.ptr;
      }
    }
    const uint16_t *tab = nullptr;
    if (epi == 1 && pk_gelu_table(&tab) != PK_OK) {
      error = std::string("GELU table: ") + pk_last_error();
      return false;
    }
    pk_i8s_args a{p->A, p->Wq, p->scale, static_cast<float *>(ws), p->C, epi == 2 ? p->residual : nullptr, tab,
                  p->M, p->N, p->K, splits, split_steps, slices * splits};
    if (!ModuleLaunch(mod->fns[0], (unsigned)(slices * splits), (unsigned)mblocks, 64u * c.num_warps, p->stream, a,
                      "pk_int8_stream", error))
      return false;
    if (splits > 1) {
      const long long groups = (long long)p->M * p->N / 8;
      constexpr long long T = PK_I8_REDUCE_THREADS;
      const unsigned blocks = (unsigned)std::min<long long>((groups + T - 1) / T, 4096);
      if (!ModuleLaunch(mod->fns[1], blocks, 1, (unsigned)T, p->stream, a, "pk_int8_reduce", error)) return false;
    }
    return true;
  };
}

// GEMM-family code objects (pk_gemm): the launch geometry follows from the
// config -- block_m x block_n tiles, 64 * num_warps threads -- and the
// operand checks are the linked path's for the same config (gemm.hip
// gemm_run_config): the DMA-ring kernel (block_k 32) and 16-byte loads
// (vector_width 8) need 16-byte aligned operands, the DMA kernel also an
// aligned C, residual and bias.
LaunchFn CodeObjectGemmLauncher(int epi, std::shared_ptr<ModuleTable> table) {
  return [epi, table](const CacheEntry &e, void *io, std::string &error) {
    MatmulIO *p = Cast<MatmulIO>(io, error);
    if (!p) return false;
    const uint16_t *R = epi == 2 ? p->residual : nullptr;
    if (!p->A || !p->B || !p->C || (epi == 1 && !p->bias) || (epi == 2 && !R)) {
      error = std::string(e.op) + " code object: null tensor pointer";
      return false;
    }
    if (!CheckEntry(e, p->M, p->N, p->K, error)) return false;
    const Config &c = e.best;
    const bool dma = c.block_k == 32;
    const bool vec = dma || c.vector_width == 8;
    if (vec && !(Aligned16(p->A) && Aligned16(p->B))) {
      error = "code-object GEMM config {" + autotune::ToString(c) + "} needs 16-byte aligned A and B";
      return false;
    }
    const uint16_t *bias = epi == 0 ? nullptr : p->bias;
    if (dma && !(Aligned16(p->C) && (!R || Aligned16(R)) && (!bias || Aligned16(bias)))) {
      error = "code-object GEMM config {" + autotune::ToString(c) + "} needs 16-byte aligned C, residual and bias";
      return false;
    }
    const std::optional<CachedBinary> bin = table->cache.GetBinary(e.gpu, e.op, e.shape);
    if (!bin) {
      error = "no code object cached for " + FormatKey(e.gpu, e.op, e.shape) +
              "; emit one (python -m polykernel_amd.emit)";
      return false;
    }
    ModuleTable::Loaded *mod = table->Get(*bin, {"pk_gemm"}, error);
    if (!mod) return false;
    const uint16_t *tab = nullptr;
    if (epi == 1 && pk_gelu_table(&tab) != PK_OK) {
      error = std::string("GELU table: ") + pk_last_error();
      return false;
    }
    pk_gemm_args a{p->A, p->B, p->C, bias, R, tab, p->M, p->N, p->K};
    unsigned tiles = 0;
    if (!TileGrid(p->M, p->N, p->K, c.block_m, c.block_n, tiles, error)) return false;
    return ModuleLaunch(mod->fns[0], tiles, 1, 64u * c.num_warps, p->stream, a, "pk_gemm", error);
  };
}

// The code object cached for an entry, or an error naming how to emit one.
std::optional<CachedBinary> BinaryOf(const ModuleTable &table, const CacheEntry &e, std::string &error) {
  std::optional<CachedBinary> bin = table.cache.GetBinary(e.gpu, e.op, e.shape);
  if (!bin)
    error = "no code object cached for " + FormatKey(e.gpu, e.op, e.shape) +
            "; emit one (python -m polykernel_amd.emit)";
  return bin;
}

// Launch a row object (pk_row, pk_row_any) on a [rows, cols] argument block
// as rowwise.hip's dispatchers launch the linked kernels: the config's
// vector kernel when it is one (vector_width 8) and the operands are 16-byte
// aligned with cols % 8 == 0 -- 4 rows per 256-thread block (block_m 4) or a
// row per block of num_warps waves -- else the generic kernel, a row per
// 256-thread block.
bool RowLaunch(ModuleTable::Loaded *mod, const Config &c, pk_row_args a, void *stream, std::string &error) {
  const bool vec = c.vector_width == 8 && a.cols % 8 == 0 && Aligned16(a.in) && Aligned16(a.out) &&
                   (!a.aux || Aligned16(a.aux)) && (!a.gamma || Aligned16(a.gamma));
  const unsigned grid = vec && c.block_m == 4 ? (unsigned)(a.rows / 4 + (a.rows % 4 != 0)) : (unsigned)a.rows;
  const unsigned threads = vec && c.block_m == 1 ? 64u * (unsigned)c.num_warps : 256u;
  return ModuleLaunch(mod->fns[vec ? 0 : 1], grid, 1, threads, stream, a, vec ? "pk_row" : "pk_row_any", error);
}

// Row-op code objects: residual + RMSNorm and masked softmax.
LaunchFn CodeObjectRowLauncher(bool softmax, std::shared_ptr<ModuleTable> table) {
  return [softmax, table](const CacheEntry &e, void *io, std::string &error) {
    pk_row_args a{};
    void *stream = nullptr;
    if (softmax) {
      SoftmaxMaskIO *p = Cast<SoftmaxMaskIO>(io, error);
      if (!p) return false;
      if (!p->logits || !p->mask || !p->out) {
        error = "fused_softmax_mask code object: null tensor pointer";
        return false;
      }
      if (!CheckEntry(e, p->rows, p->cols, 0, error)) return false;
      a = pk_row_args{p->logits, p->mask, nullptr, p->out, p->rows, p->cols, 0.f, 0.f};
      stream = p->stream;
    } else {
      ResidualRmsnormIO *p = Cast<ResidualRmsnormIO>(io, error);
      if (!p) return false;
      if (!p->x || !p->r || !p->out) {
        error = "fused_residual_rmsnorm code object: null tensor pointer";
        return false;
      }
      if (!CheckEntry(e, p->rows, p->cols, 0, error)) return false;
      a = pk_row_args{p->x, p->r, p->gamma, p->out, p->rows, p->cols, 1.0f / (float)p->cols, p->eps};
      stream = p->stream;
    }
    const std::optional<CachedBinary> bin = BinaryOf(*table, e, error);
    if (!bin) return false;
    ModuleTable::Loaded *mod = table->Get(*bin, {"pk_row", "pk_row_any"}, error);
    if (!mod) return false;
    return RowLaunch(mod, e.best, a, stream, error);
  };
}

// RMSNorm -> MatMul code objects.  The panel config (pk_panel): the operand
// conditions and the LDS size of gemm.hip fused_rmsnorm_matmul for that
// kernel.  A GEMM config: RMSNorm into library workspace (pk_row /
// pk_row_any at the (M, K) row config), then pk_gemm with that config's
// operand checks.
LaunchFn CodeObjectPanelLauncher(std::shared_ptr<ModuleTable> table) {
  return [table](const CacheEntry &e, void *io, std::string &error) {
    RmsnormMatmulIO *p = Cast<RmsnormMatmulIO>(io, error);
    if (!p) return false;
    if (!p->x || !p->W || !p->out) {
      error = "fused_rmsnorm_matmul code object: null tensor pointer";
      return false;
    }
    if (!CheckEntry(e, p->M, p->N, p->K, error)) return false;
    const Config &c = e.best;
    if (IsPanelConfig(c, p->K)) {
      if (!Aligned16(p->x) || !Aligned16(p->W) || (p->gamma && !Aligned16(p->gamma)) || !Aligned16(p->out)) {
        error = "code-object RMSNorm -> MatMul panel config {" + autotune::ToString(c) +
                "} needs 16-byte aligned x, W, gamma and out";
        return false;
      }
      const std::optional<CachedBinary> bin = BinaryOf(*table, e, error);
      if (!bin) return false;
      ModuleTable::Loaded *mod = table->Get(*bin, {"pk_panel"}, error);
      if (!mod) return false;
      pk_panel_args a{p->x, p->gamma, p->W, p->out, p->M, p->N, p->K, 1.0f / (float)p->K, p->eps};
      unsigned tiles = 0;
      if (!TileGrid(p->M, p->N, p->K, 32, 64, tiles, error)) return false;
      return ModuleLaunch(mod->fns[0], tiles, 1, (unsigned)PK_PANEL_THREADS, p->stream, a, "pk_panel", error,
                          pk_panel_lds_bytes(p->K));
    }
    // GEMM config: the row normalisation, then the plain GEMM
    const bool dma = c.block_k == 32;
    if ((dma || c.vector_width == 8) && !Aligned16(p->W)) {
      error = "code-object GEMM config {" + autotune::ToString(c) + "} needs a 16-byte aligned W";
      return false;
    }
    if (dma && !Aligned16(p->out)) {
      error = "code-object GEMM config {" + autotune::ToString(c) + "} needs a 16-byte aligned out";
      return false;
    }
    pk_config rc{};
    if (pk_op_default_config("fused_residual_rmsnorm", p->M, p->K, 0, &rc) != PK_OK) {
      error = std::string("row config: ") + pk_last_error();
      return false;
    }
    const std::optional<CachedBinary> bin = BinaryOf(*table, e, error);
    if (!bin) return false;
    ModuleTable::Loaded *mod = table->Get(*bin, {"pk_row", "pk_row_any", "pk_gemm"}, error);
    if (!mod) return false;
    WorkspaceLease lease;  // the normalised rows, held until the GEMM is queued
    if (library_workspace((size_t)p->M * p->K * 2, p->stream, lease) != PK_OK) {
      error = std::string("library workspace: ") + pk_last_error();
      return false;
    }
    uint16_t *xn = static_cast<uint16_t *>(lease.ptr);
    const Config row{rc.block_m, rc.block_n, rc.block_k, rc.num_warps, rc.vector_width, rc.unroll,
                     rc.shared_memory_stages};
    if (!RowLaunch(mod, row, pk_row_args{p->x, nullptr, p->gamma, xn, p->M, p->K, 1.0f / (float)p->K, p->eps},
                   p->stream, error))
      return false;
    pk_gemm_args g{xn, p->W, p->out, nullptr, nullptr, nullptr, p->M, p->N, p->K};
    unsigned tiles = 0;
    if (!TileGrid(p->M, p->N, p->K, c.block_m, c.block_n, tiles, error)) return false;
    return ModuleLaunch(mod->fns[2], tiles, 1, 64u * c.num_warps, p->stream, g, "pk_gemm", error);
  };
}

// Attention code objects: the library's attention dispatcher makes the same
// tile-shape, key-split, workspace and append decisions as for the linked
// kernels and launches the object's entry points (attention_module.hpp).
LaunchFn CodeObjectAttentionLauncher(std::shared_ptr<ModuleTable> table) {
  return [table](const CacheEntry &e, void *io, std::string &error) {
    KvAppendAttentionIO *p = Cast<KvAppendAttentionIO>(io, error);
    if (!p) return false;
    if (!p->Q || !p->Kc || !p->Vc || !p->O || (p->S_q > 0 && (!p->Kn || !p->Vn))) {
      error = "fused_kv_append_attention code object: null tensor pointer";
      return false;
    }
    if (!CheckEntry(e, p->S_q, (std::int64_t)p->S_cache + p->S_q, p->D, error)) return false;
    const std::optional<CachedBinary> bin = table->cache.GetBinary(e.gpu, e.op, e.shape);
    if (!bin) {
      error = "no code object cached for " + FormatKey(e.gpu, e.op, e.shape) +
              "; emit one (python -m polykernel_amd.emit)";
      return false;
    }
    const bool flash = e.best.num_warps == 8;
    ModuleTable::Loaded *m =
        flash ? table->Get(*bin, {"pk_fa_fused", "pk_fa_combine"}, error)
              : table->Get(*bin, {"pk_att", "pk_att_unaligned", "pk_att_combine", "pk_kv_append"}, error);
    if (!m) return false;
    AttModule mod;
    if (flash) {
      mod.fa_fused = m->fns[0];
      mod.fa_combine = m->fns[1];
    } else {
      mod.att = m->fns[0];
      mod.att_unaligned = m->fns[1];
      mod.att_combine = m->fns[2];
      mod.kv_append = m->fns[3];
    }
    const pk_config cfg = ToPk(e.best);
    return Launched(fused_kv_append_attention_module(p->Q, p->Kc, p->Vc, p->Kn, p->Vn, p->O, p->B, p->H, p->S_q,
                                                     p->S_cache, p->D, p->cache_capacity, p->scale, p->causal, &cfg,
                                                     &mod, p->stream),
                    e, error);
  };
}

}  // namespace

void RegisterCodeObjectLaunchers(Runtime &rt, const KernelCache &cache) {
  auto table = std::make_shared<ModuleTable>(cache);
  rt.RegisterLauncher("fused_kv_append_attention", CodeObjectAttentionLauncher(table));
  rt.RegisterLauncher("matmul", CodeObjectGemmLauncher(0, table));
  rt.RegisterLauncher("fused_matmul_bias_gelu", CodeObjectGemmLauncher(1, table));
  rt.RegisterLauncher("fused_matmul_bias_residual", CodeObjectGemmLauncher(2, table));
  rt.RegisterLauncher("matmul_int8", CodeObjectInt8Launcher(0, table));
  rt.RegisterLauncher("matmul_int8_gelu", CodeObjectInt8Launcher(1, table));
  rt.RegisterLauncher("matmul_int8_residual", CodeObjectInt8Launcher(2, table));
  rt.RegisterLauncher("fused_residual_rmsnorm", CodeObjectRowLauncher(false, table));
  rt.RegisterLauncher("fused_softmax_mask", CodeObjectRowLauncher(true, table));
  rt.RegisterLauncher("fused_rmsnorm_matmul", CodeObjectPanelLauncher(table));
}

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
    // the entry's config; operands that are not 16-byte aligned take the generic kernel
    const pk_config cfg = ToPk(e.best);
    const bool aligned = Aligned16(p->x) && Aligned16(p->r) && Aligned16(p->out) && (!p->gamma || Aligned16(p->gamma));
    return Launched(pk_fused_residual_rmsnorm_config(p->x, p->r, p->gamma, p->out, p->rows, p->cols, p->eps,
                                                     aligned ? &cfg : nullptr, p->stream),
                    e, error);
  });
  rt.RegisterLauncher("fused_softmax_mask", [](const CacheEntry &e, void *io, std::string &error) {
    SoftmaxMaskIO *p = Cast<SoftmaxMaskIO>(io, error);
    if (!p || !CheckEntry(e, p->rows, p->cols, 0, error)) return false;
    const pk_config cfg = ToPk(e.best);
    const bool aligned = Aligned16(p->logits) && Aligned16(p->mask) && Aligned16(p->out);
    return Launched(pk_fused_softmax_mask_config(p->logits, p->mask, p->out, p->rows, p->cols,
                                                 aligned ? &cfg : nullptr, p->stream),
                    e, error);
  });
  rt.RegisterLauncher("fused_kv_append_attention", [](const CacheEntry &e, void *io, std::string &error) {
    KvAppendAttentionIO *p = Cast<KvAppendAttentionIO>(io, error);
    if (!p || !CheckEntry(e, p->S_q, (std::int64_t)p->S_cache + p->S_q, p->D, error)) return false;
    const pk_config cfg = ToPk(e.best);
    return Launched(pk_fused_kv_append_attention_config(p->Q, p->Kc, p->Vc, p->Kn, p->Vn, p->O, p->B, p->H, p->S_q,
                                                        p->S_cache, p->D, p->cache_capacity, p->scale, p->causal,
                                                        &cfg, p->stream),
                    e, error);
  });
}

}  // namespace pk::runtime
