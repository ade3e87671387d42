// internal.hpp -- helpers shared by the runtime's translation units.
#pragma once

#include "../../../include/polykernel_amd_runtime.hpp"
#include "json.hpp"

namespace pk::autotune::detail {

json::Value ConfigJson(const Config &c);
json::Value CorrectnessJson(const Correctness &c);
json::Value EntryJson(const CacheEntry &e);

}  // namespace pk::autotune::detail

namespace pk {
// Thread-local error message of the C-ABI (pk_last_error).
void set_error(const char *fmt, ...);
void clear_error();
}  // namespace pk
