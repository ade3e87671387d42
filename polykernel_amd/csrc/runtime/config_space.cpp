// config_space.cpp -- the gfx950 tuning space: the configurations the
// kernels implement for an op and shape, pruned by the CU's limits.
//
// The reference enumerates a generic 4608-point tile grid and prunes it with
// sm_90 limits (lib/Autotune/ConfigSpace.cpp:33-120).  Here the kernels
// themselves list the variants they were written for (pk_op_configs, each
// family beside its dispatcher), so every candidate is one that runs; the
// pruner then applies the MI355X limits -- 64-lane waves, at most 1024
// threads per workgroup, 160 KiB of LDS per CU -- which matter when a caller
// tunes for a smaller budget (e.g. to leave LDS for a co-resident kernel).
#include <algorithm>
#include <cstring>

#include "../../../include/polykernel_amd_runtime.hpp"
#include "internal.hpp"

namespace pk::autotune {

namespace {

enum class Family { Unknown, Gemm, Int8, RmsnormMatmul, Rowwise, Softmax, Attention };

Family FamilyOf(std::string_view op) {
  if (op == "matmul" || op == "fused_matmul_bias_gelu" || op == "fused_matmul_bias_residual") return Family::Gemm;
  if (op == "matmul_int8" || op == "matmul_int8_gelu" || op == "matmul_int8_residual") return Family::Int8;
  if (op == "fused_rmsnorm_matmul") return Family::RmsnormMatmul;
  if (op == "fused_residual_rmsnorm") return Family::Rowwise;
  if (op == "fused_softmax_mask") return Family::Softmax;
  if (op == "fused_kv_append_attention") return Family::Attention;
  return Family::Unknown;
}

const char *DtypeOf(Family f) {
  switch (f) {
    case Family::Int8: return "int8";
    case Family::Softmax: return "fp32";
    case Family::Unknown: return "";
    default: return "bf16";
  }
}

Config FromPk(const pk_config &c) {
  return Config{c.block_m, c.block_n, c.block_k, c.num_warps, c.vector_width, c.unroll, c.shared_memory_stages};
}

}  // namespace

const std::vector<std::string> &BuiltinOps() {
  static const std::vector<std::string> ops = {
      "matmul",           "fused_matmul_bias_gelu", "fused_matmul_bias_residual", "matmul_int8",
      "matmul_int8_gelu", "matmul_int8_residual",   "fused_rmsnorm_matmul",       "fused_residual_rmsnorm",
      "fused_softmax_mask", "fused_kv_append_attention"};
  return ops;
}

Shape OpShape(std::string_view op, std::int64_t m, std::int64_t n, std::int64_t k) {
  return Shape{m, n, k, DtypeOf(FamilyOf(op))};
}

long long ConfigSpace::LdsBytes(std::string_view op, const Shape &shape, const Config &c) {
  switch (FamilyOf(op)) {
    case Family::Gemm:
      return 2LL * c.shared_memory_stages * ((long long)c.block_m * c.block_k + (long long)c.block_k * c.block_n);
    case Family::Int8: {
      if (c.num_warps <= 0) return 0;
      const long long nt = c.block_n / (16LL * c.num_warps), mt = c.block_m / 16;
      return (long long)c.shared_memory_stages * c.num_warps * 1024LL * (nt + 2 * mt);
    }
    case Family::RmsnormMatmul:
      // whole-K kernel: W slice (K x 64) + normalised panel (32 x K)
      if (runtime::IsPanelConfig(c, shape.k)) return pk_panel_lds_bytes((int)shape.k);
      return 2LL * c.shared_memory_stages * ((long long)c.block_m * c.block_k + (long long)c.block_k * c.block_n);
    case Family::Attention:
      // K/V ring + the query-group merge buffer it aliases
      return c.shared_memory_stages * 2LL * c.block_n * c.block_k * 2;
    case Family::Rowwise:
    case Family::Softmax:
      return 64;  // cross-wave reduction slots
    default:
      return 0;
  }
}

std::string ConfigSpace::RejectionReason(std::string_view op, const Shape &shape, const Config &c,
                                         const ArchLimits &limits) {
  if (FamilyOf(op) == Family::Unknown) return "unknown op";
  if (c.num_warps <= 0 || (long long)c.num_warps * limits.wave_size > limits.max_threads_per_workgroup)
    return "num_warps * wave_size must be in 1..max_threads_per_workgroup";
  if (c.block_m <= 0 || c.block_n <= 0) return "block_m and block_n must be positive";
  if (c.vector_width <= 0 || c.unroll <= 0 || c.shared_memory_stages <= 0)
    return "vector_width, unroll and shared_memory_stages must be positive";
  if (LdsBytes(op, shape, c) > limits.lds_per_cu_bytes) return "LDS footprint exceeds lds_per_cu_bytes";
  return {};
}

std::vector<Config> ConfigSpace::Candidates(std::string_view op, const Shape &shape, const ArchLimits &limits) {
  const Family f = FamilyOf(op);
  if (f == Family::Unknown || shape.dtype != DtypeOf(f)) return {};
  const std::string name(op);
  const int total = pk_op_configs(name.c_str(), shape.m, shape.n, shape.k, nullptr, 0);
  if (total <= 0) return {};
  std::vector<pk_config> raw(total);
  const int got = pk_op_configs(name.c_str(), shape.m, shape.n, shape.k, raw.data(), total);
  std::vector<Config> out;
  for (int i = 0; i < std::min(got, total); ++i) {
    const Config c = FromPk(raw[i]);
    if (IsAdmissible(op, shape, c, limits) && std::find(out.begin(), out.end(), c) == out.end()) out.push_back(c);
  }
  return out;
}

std::optional<Config> ConfigSpace::Default(std::string_view op, const Shape &shape) {
  const Family f = FamilyOf(op);
  if (f == Family::Unknown || shape.dtype != DtypeOf(f)) return std::nullopt;
  pk_config c{};
  if (pk_op_default_config(std::string(op).c_str(), shape.m, shape.n, shape.k, &c) != PK_OK) return std::nullopt;
  return FromPk(c);
}

}  // namespace pk::autotune
