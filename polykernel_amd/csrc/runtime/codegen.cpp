// codegen.cpp -- the gfx950 emitter: a tuned cache entry becomes a standalone
// code object (.hsaco) that the runtime loads with hipModuleLoad.
//
// The reference lowers its IR ops to generic HIP/CUDA source
// (lib/Codegen/LowerToHip.cpp) and compiles per-op shared libraries.  Here the
// kernels already exist as templates written for gfx950; emitting a tuned
// variant means instantiating the template at the entry's configuration
// behind extern "C" entry points with fixed names, and compiling that one
// translation unit for gfx950 with hipcc --genco.  The code object's FNV-1a
// hash goes into the KernelCache beside the entry, so a code object that
// changes on disk is refused (CodeObject::Load) and dropped
// (KernelCache::InvalidateStale).
//
// Emitted entry points:
//   matmul_int8, matmul_int8_gelu, matmul_int8_residual (int8_stream.hpp):
//     pk_int8_stream(pk_i8s_args)  grid (slices * splits, m-blocks), 64 * num_warps threads
//     pk_int8_reduce(pk_i8s_args)  the split reduction, PK_I8_REDUCE_THREADS threads
//   matmul, fused_matmul_bias_gelu, fused_matmul_bias_residual (gemm_kernels.hpp):
//     pk_gemm(pk_gemm_args)        grid ceil(M/block_m) * ceil(N/block_n), 64 * num_warps threads;
//                                  block_k 32: the DMA-ring kernel at shared_memory_stages,
//                                  block_k 64: the register-staged kernel (vector_width 8:
//                                  16-byte loads, 1: element loads)
//   fused_kv_append_attention (attention_kernels.hpp), the flash kernel's tile shapes (num_warps 8):
//     pk_fa_fused(pk_fa_args)      the flash kernel with the in-place append, 512 threads
//     pk_fa_combine(pk_fa_args)    the merge of key splits, 256 threads
//   and the generic kernel (num_warps 4, block_k = padded head dim; 1024:
//   the wide-head kernel for head dims 257..1024):
//     pk_att / pk_att_unaligned(pk_att_args), pk_att_combine(pk_att_args),
//     pk_kv_append(pk_kv_append_args)
//   The runtime hands these to the library's attention dispatcher
//   (attention_module.hpp), which makes the linked path's tile-shape, key-split
//   and workspace decisions and launches the object's entry points.
//   fused_residual_rmsnorm, fused_softmax_mask (rowwise_kernels.hpp):
//     pk_row(pk_row_args)          the config's row kernel: vector_width 8 -- one wave per row
//                                  (block_m 4, grid ceil(rows/4), 256 threads) or num_warps waves
//                                  per row (block_m 1, grid rows, 64 * num_warps threads, 4/8/16)
//                                  with `unroll` 16-byte vectors per lane; vector_width 1 -- the
//                                  generic kernel (grid rows, 256 threads)
//     pk_row_any(pk_row_args)      the generic kernel, for operands the vector kernel cannot take
//   fused_rmsnorm_matmul (gemm_kernels.hpp, rowwise_kernels.hpp):
//     pk_panel(pk_panel_args)      block_k = K: the whole-K panel kernel (256 threads); grid
//                                  ceil(M/32) * ceil(N/64), dynamic LDS as in gemm.hip
//   or, for a GEMM config (every other shape): the row normalisation into workspace
//     pk_row / pk_row_any(pk_row_args) (RMSNorm with gamma at the (M, K) row config), then
//     pk_gemm(pk_gemm_args)        the config's GEMM kernel
#include <fcntl.h>
#include <spawn.h>
#include <sys/wait.h>
#include <unistd.h>

#include <algorithm>
#include <cstdlib>
#include <cstring>
#include <filesystem>
#include <fstream>
#include <sstream>

#include "internal.hpp"

extern char **environ;

namespace pk::codegen {

using autotune::CacheEntry;
using autotune::Config;

namespace {

int Int8Epilogue(const std::string &op) {
  if (op == "matmul_int8") return 0;
  if (op == "matmul_int8_gelu") return 1;
  if (op == "matmul_int8_residual") return 2;
  return -1;
}

// Epilogue of a GEMM-family op (gemm_kernels.hpp Epi); the residual op's
// object serves calls without a bias too (the kernels read a null bias as 0).
int GemmEpilogue(const std::string &op) {
  if (op == "matmul") return 0;
  if (op == "fused_matmul_bias_gelu") return 1;
  if (op == "fused_matmul_bias_residual") return 2;
  return -1;
}

// The kernel template a GEMM config instantiates (the variants of
// gemm.hip gemm_variant_config): returns false for a config it does not know.
bool GemmInstance(const Config &c, int epi, std::string &body, int &threads) {
  threads = 64 * c.num_warps;
  if (c.block_k == 32 && c.block_m == 256 && c.block_n == 256 && c.num_warps == 8 &&
      (c.shared_memory_stages == 4 || c.shared_memory_stages == 5)) {
    body = "pk::gk::gemm_dma_body<" + std::to_string(epi) + ", " + std::to_string(c.shared_memory_stages) + ", 8, 4>";
    return true;
  }
  if (c.block_k != 64 || (c.vector_width != 8 && c.vector_width != 1)) return false;
  int wm = 0, wn = 0;
  if (c.block_m == 256 && c.block_n == 256 && c.num_warps == 8) wm = 2, wn = 4;
  else if ((c.block_m == 128 || c.block_m == 64) && c.block_n == c.block_m && c.num_warps == 4) wm = 2, wn = 2;
  else return false;
  body = "pk::gk::gemm_reg_body<" + std::to_string(c.block_m) + ", " + std::to_string(c.block_n) + ", " +
         std::to_string(wm) + ", " + std::to_string(wn) + ", " + std::to_string(epi) + ", " +
         (c.vector_width == 8 ? "true" : "false") + ">";
  return true;
}

// The row kernel a config instantiates (rowwise.hip rmsnorm_dispatch and
// softmax_dispatch): vector_width 8 -- NW waves per row (block_m 4: one, 1:
// four) with VPT = unroll vectors per lane; vector_width 1 -- the generic
// kernel.  `kind` is the third template argument: RMSNorm's residual flag
// ("true" / "false") or softmax's mode ("1": masked).
// The row kernel a config names: waves per row = 1 (block_m 4: 4 rows per
// 256-thread block) or num_warps (block_m 1: a row per num_warps * 64 threads,
// 4, 8 or 16), unroll 16-byte vectors per lane; `threads` = the pk_row block size.
bool RowInstance(const Config &c, bool softmax, const std::string &kind, std::string &body, std::string &any,
                 int &threads) {
  const std::string ns = softmax ? "pk::row::softmax_" : "pk::row::rmsnorm_";
  any = ns + "generic_body<" + kind + ">";
  threads = 256;
  if (c.block_k != 0) return false;
  if (c.vector_width == 1) {
    body = any;
    return c.num_warps == 4;
  }
  if (c.vector_width != 8 || c.unroll < 1 || c.unroll > 16) return false;
  if (c.block_m == 4 && c.num_warps == 4) {
    body = ns + "vec_body<1, " + std::to_string(c.unroll) + ", " + kind + ">";
    return true;
  }
  if (c.block_m != 1 || (c.num_warps != 4 && c.num_warps != 8 && c.num_warps != 16) || c.unroll > 16) return false;
  threads = 64 * c.num_warps;
  if (c.num_warps == 16 && c.unroll == 16)  // rows held as packed bf16
    body = ns + "packed_body<" + kind + ">";
  else
    body = ns + "vec_body<" + std::to_string(c.num_warps) + ", " + std::to_string(c.unroll) + ", " + kind + ">";
  return true;
}

std::string RowEntryPoints(const std::string &body, const std::string &any, int threads) {
  return "extern \"C\" __global__ __launch_bounds__(" + std::to_string(threads) +
         ") void pk_row(pk_row_args a) {\n  " + body +
         "(a);\n}\n\nextern \"C\" __global__ __launch_bounds__(256) void pk_row_any(pk_row_args a) {\n  " + any +
         "(a);\n}\n";
}

std::string Hipcc() {
  if (const char *p = std::getenv("HIPCC")) return p;
  const char *rocm = std::getenv("ROCM_PATH");
  return std::string(rocm ? rocm : "/opt/rocm") + "/bin/hipcc";
}

// Run argv[0] with argv as a child process; its output goes to `log`.
bool RunChild(const std::vector<std::string> &argv, const std::string &log, std::string &error) {
  std::vector<char *> args;
  for (const std::string &a : argv) args.push_back(const_cast<char *>(a.c_str()));
  args.push_back(nullptr);
  posix_spawn_file_actions_t fa;
  posix_spawn_file_actions_init(&fa);
  posix_spawn_file_actions_addopen(&fa, 1, log.c_str(), O_WRONLY | O_CREAT | O_TRUNC, 0644);
  posix_spawn_file_actions_adddup2(&fa, 1, 2);
  pid_t pid = 0;
  const int rc = posix_spawnp(&pid, args[0], &fa, nullptr, args.data(), environ);
  posix_spawn_file_actions_destroy(&fa);
  if (rc != 0) {
    error = "cannot start " + argv[0] + ": " + std::strerror(rc);
    return false;
  }
  int status = 0;
  if (waitpid(pid, &status, 0) < 0 || !WIFEXITED(status) || WEXITSTATUS(status) != 0) {
    std::ifstream in(log);
    std::stringstream ss;
    ss << in.rdbuf();
    std::string out = ss.str();
    if (out.size() > 4000) out = out.substr(out.size() - 4000);
    error = argv[0] + " failed (status " + std::to_string(status) + "):\n" + out;
    return false;
  }
  return true;
}

}  // namespace

bool EmitSource(const CacheEntry &e, std::string &source, std::string &error) {
  const int epi = Int8Epilogue(e.op), gepi = GemmEpilogue(e.op);
  const bool attention = e.op == "fused_kv_append_attention";
  const bool rms = e.op == "fused_residual_rmsnorm", smx = e.op == "fused_softmax_mask";
  const bool panel = e.op == "fused_rmsnorm_matmul";
  if (epi < 0 && gepi < 0 && !attention && !rms && !smx && !panel) {
    error = "the emitter instantiates the ops of the tuning cache (matmul, fused_matmul_bias_gelu, "
            "fused_matmul_bias_residual, matmul_int8, matmul_int8_gelu, matmul_int8_residual, "
            "fused_rmsnorm_matmul, fused_residual_rmsnorm, fused_softmax_mask, fused_kv_append_attention), "
            "not " +
            e.op;
    return false;
  }
  const std::vector<Config> cands = autotune::ConfigSpace::Candidates(e.op, e.shape);
  if (std::find(cands.begin(), cands.end(), e.best) == cands.end()) {
    error = "config {" + autotune::ToString(e.best) + "} is not one the gfx950 kernels implement for " +
            runtime::FormatKey(e.gpu, e.op, e.shape);
    return false;
  }
  if (e.gpu != "gfx950") {
    error = "the emitter targets gfx950, not " + e.gpu;
    return false;
  }
  const Config &c = e.best;
  const std::string head = "// Emitted by the polykernel_amd gfx950 emitter for " + runtime::FormatKey(e.gpu, e.op, e.shape) +
                           "\n// config: " + autotune::ToString(c) + "\n";
  if (rms || smx) {
    std::string body, any;
    int threads = 0;
    if (!RowInstance(c, smx, smx ? "1" : "true", body, any, threads)) {
      error = "config {" + autotune::ToString(c) + "} has no row kernel template";
      return false;
    }
    source = head + "#include \"rowwise_kernels.hpp\"\n\n" + RowEntryPoints(body, any, threads);
    return true;
  }
  if (panel) {
    if (runtime::IsPanelConfig(c, e.shape.k)) {  // whole-K panel kernel
      source = head + "#include \"gemm_kernels.hpp\"\n\n" +
               "extern \"C\" __global__ __launch_bounds__(" + std::to_string(PK_PANEL_THREADS) +
               ") void pk_panel(pk_panel_args a) {\n"
               "  pk::gk::rmsnorm_panel_fast_body(a);\n}\n";
      return true;
    }
    // rows too long for a panel: RMSNorm (with gamma) at the (M, K) row
    // config into workspace, then the config's GEMM
    pk_config rc{};
    std::string rbody, rany, gbody;
    int threads = 0, rthreads = 0;
    if (pk_op_default_config("fused_residual_rmsnorm", e.shape.m, e.shape.k, 0, &rc) != PK_OK ||
        !RowInstance(Config{rc.block_m, rc.block_n, rc.block_k, rc.num_warps, rc.vector_width, rc.unroll,
                            rc.shared_memory_stages},
                     false, "false", rbody, rany, rthreads) ||
        !GemmInstance(c, 0, gbody, threads)) {
      error = "config {" + autotune::ToString(c) + "} has no RMSNorm -> GEMM kernel template";
      return false;
    }
    source = head + "#include \"gemm_kernels.hpp\"\n#include \"rowwise_kernels.hpp\"\n\n" +
             RowEntryPoints(rbody, rany, rthreads) + "\nextern \"C\" __global__ __launch_bounds__(" + std::to_string(threads) +
             (c.block_k == 32 ? ", 1" : "") + ") void pk_gemm(pk_gemm_args g) {\n  " + gbody + "(g);\n}\n";
    return true;
  }
  if (attention) {
    const int dp = c.block_k;
    std::ostringstream s;
    s << "// Emitted by the polykernel_amd gfx950 emitter for " << runtime::FormatKey(e.gpu, e.op, e.shape) << "\n"
      << "// config: " << autotune::ToString(c) << "\n"
      << "#include \"attention_kernels.hpp\"\n\n";
    if (c.num_warps == 8) {  // the flash kernel at this tile shape
      const int qg = c.block_m / 32;
      s << "extern \"C\" __global__ __launch_bounds__(512, 1) void pk_fa_fused(pk_fa_args g) {\n"
        << "  pk::att::fa_body<" << dp << ", " << qg << ", true>(g);\n}\n\n"
        << "extern \"C\" __global__ __launch_bounds__(256) void pk_fa_combine(pk_fa_args g) {\n"
        << "  pk::att::fa_combine_body<" << dp << ">(g);\n}\n";
    } else {
      // block_k 1024: the wide-head kernel (head dims split over the waves, one wave per SIMD)
      const bool wide = dp == 1024;
      const std::string body = wide ? "pk::att::att_wide_body<" : "pk::att::att_body<" + std::to_string(dp) + ", ";
      const std::string bounds = wide ? "256, 1" : "256";
      s << "extern \"C\" __global__ __launch_bounds__(" << bounds << ") void pk_att(pk_att_args g) {\n"
        << "  " << body << "true>(g);\n}\n\n"
        << "extern \"C\" __global__ __launch_bounds__(" << bounds << ") void pk_att_unaligned(pk_att_args g) {\n"
        << "  " << body << "false>(g);\n}\n\n"
        << "extern \"C\" __global__ __launch_bounds__(256) void pk_att_combine(pk_att_args g) {\n"
        << "  pk::att::att_combine_body<" << dp << ">(g);\n}\n\n"
        << "extern \"C\" __global__ __launch_bounds__(256) void pk_kv_append(pk_kv_append_args a) {\n"
        << "  pk::att::kv_append_body(a);\n}\n";
    }
    source = s.str();
    return true;
  }
  if (gepi >= 0) {
    std::string body;
    int threads = 0;
    if (!GemmInstance(c, gepi, body, threads)) {
      error = "config {" + autotune::ToString(c) + "} has no GEMM kernel template";
      return false;
    }
    std::ostringstream s;
    s << "// Emitted by the polykernel_amd gfx950 emitter for " << runtime::FormatKey(e.gpu, e.op, e.shape) << "\n"
      << "// config: " << autotune::ToString(c) << "\n"
      << "#include \"gemm_kernels.hpp\"\n\n"
      << "extern \"C\" __global__ __launch_bounds__(" << threads << (c.block_k == 32 ? ", 1" : "")
      << ") void pk_gemm(pk_gemm_args g) {\n"
      << "  " << body << "(g);\n}\n";
    source = s.str();
    return true;
  }
  const int nt = c.block_n / (16 * c.num_warps), mt = c.block_m / 16;
  std::ostringstream s;
  s << "// Emitted by the polykernel_amd gfx950 emitter for " << runtime::FormatKey(e.gpu, e.op, e.shape) << "\n"
    << "// config: " << autotune::ToString(c) << "\n"
    << "#include \"int8_stream.hpp\"\n\n"
    << "extern \"C\" __global__ __launch_bounds__(" << 64 * c.num_warps << ", 1) void pk_int8_stream(pk_i8s_args g) {\n"
    << "  pk::i8s::stream_body<" << nt << ", " << mt << ", " << c.num_warps << ", " << c.shared_memory_stages << ", "
    << epi << ">(g);\n}\n\n"
    << "extern \"C\" __global__ __launch_bounds__(PK_I8_REDUCE_THREADS) void pk_int8_reduce(pk_i8s_args g) {\n"
    << "  pk::i8s::reduce8_body<" << epi << ">(g.partial, g.splits, g.M, g.N, g.scale, g.R, g.gelu_tab, g.C);\n}\n";
  source = s.str();
  return true;
}

bool CompileCodeObject(const std::string &source_path, const std::string &csrc_dir, const std::string &out_path,
                       std::string &error) {
  const std::vector<std::string> argv = {Hipcc(),
                                         "--offload-arch=gfx950",
                                         "--genco",
                                         "--no-gpu-bundle-output",  // a plain ELF code object
                                         "-O3",
                                         "-std=c++17",
                                         "-Xclang",
                                         "-target-feature",
                                         "-Xclang",
                                         "-packed-fp32-ops",
                                         "-mllvm",
                                         "-pragma-unroll-threshold=1000000",
                                         "-I",
                                         csrc_dir,
                                         "-I",
                                         csrc_dir + "/../../include",
                                         source_path,
                                         "-o",
                                         out_path};
  if (!RunChild(argv, out_path + ".log", error)) return false;
  std::ifstream in(out_path, std::ios::binary);
  char magic[4] = {};
  in.read(magic, 4);
  if (!in || magic[0] != 0x7f || magic[1] != 'E' || magic[2] != 'L' || magic[3] != 'F') {
    error = out_path + " is not an ELF code object";
    return false;
  }
  return true;
}

bool EmitCodeObject(runtime::KernelCache &cache, const CacheEntry &e, const std::string &csrc_dir,
                    const std::string &out_dir, std::string &error) {
  std::string source;
  if (!EmitSource(e, source, error)) return false;
  std::error_code ec;
  std::filesystem::create_directories(out_dir, ec);
  if (ec) {
    error = "cannot create " + out_dir + ": " + ec.message();
    return false;
  }
  // one file per (op, shape, config): a re-tuned entry gets a new object
  const Config &c = e.best;
  std::ostringstream name;
  name << e.op << "_M" << e.shape.m << "_N" << e.shape.n << "_K" << e.shape.k << "_" << c.block_m << "x" << c.block_n
       << "x" << c.block_k << "_w" << c.num_warps << "_s" << c.shared_memory_stages << "_v" << c.vector_width
       << "_u" << c.unroll;
  const std::string base = std::filesystem::absolute(std::filesystem::path(out_dir) / name.str()).string();
  {
    std::ofstream out(base + ".hip");
    out << source;
    if (!out) {
      error = "cannot write " + base + ".hip";
      return false;
    }
  }
  if (!CompileCodeObject(base + ".hip", csrc_dir, base + ".hsaco", error)) return false;
  std::string hash;
  if (!runtime::HashFile(base + ".hsaco", hash, error)) return false;
  if (!cache.Put(e) || !cache.PutBinary(e.gpu, e.op, e.shape, runtime::CachedBinary{base + ".hsaco", hash})) {
    error = "cannot record the code object of " + runtime::FormatKey(e.gpu, e.op, e.shape);
    return false;
  }
  return true;
}

}  // namespace pk::codegen
