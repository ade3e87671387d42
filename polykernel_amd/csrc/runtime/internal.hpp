// internal.hpp -- helpers shared by the runtime's translation units.
#pragma once

#include "../../../include/polykernel_amd_runtime.hpp"
#include "../gemm_args.h"
#include "json.hpp"

namespace pk::autotune::detail {

json::Value ConfigJson(const Config &c);
json::Value CorrectnessJson(const Correctness &c);
json::Value EntryJson(const CacheEntry &e);

}  // namespace pk::autotune::detail

namespace pk::runtime {

// The whole-K RMSNorm -> MatMul panel config: 32 x 64 output tiles
// (RQ_BM x RQ_BN of gemm_kernels.hpp), PK_PANEL_THREADS / 64 waves and
// block_k equal to the shape's K.  No GEMM variant has a 32 x 64 tile, so the tile identifies it:
// block_k == K alone also matches a 64-deep GEMM config at K = 64.
inline bool IsPanelConfig(const autotune::Config &c, std::int64_t K) {
  return c.block_m == 32 && c.block_n == 64 && c.block_k == K && c.num_warps == PK_PANEL_THREADS / 64;
}

}  // namespace pk::runtime

namespace pk {
// Thread-local error message of the C-ABI (pk_last_error).
void set_error(const char *fmt, ...);
void clear_error();
}  // namespace pk
