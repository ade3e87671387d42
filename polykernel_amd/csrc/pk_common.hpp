// pk_common.hpp -- shared device/host helpers for the gfx950 kernels.
//
// bf16 conversions follow the reference rounding contract
// (kernels/cpu/cpu_reference.h:37-61): exact upcast, RNE downcast with
// NaN -> quiet NaN.  Error plumbing implements the C-ABI convention: return a
// negative status and keep a thread-local message, never abort.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <string>

#include "../../include/polykernel_amd.h"

namespace pk {

// ---- error state ---------------------------------------------------------
void set_error(const char *fmt, ...);
void clear_error();
int hip_fail(hipError_t e, const char *what);

#define PK_CHECK_ARG(cond, ...)                                                      \
  do {                                                                               \
    if (!(cond)) {                                                                   \
      ::pk::set_error(__VA_ARGS__);                                                  \
      return PK_ERR_INVALID_ARG;                                                     \
    }                                                                                \
  } while (0)

#define PK_HIP(call)                                                                 \
  do {                                                                               \
    hipError_t pk_e_ = (call);                                                       \
    if (pk_e_ != hipSuccess) return ::pk::hip_fail(pk_e_, #call);                    \
  } while (0)

// After a <<<>>> launch: surface configuration errors as PK_ERR_LAUNCH.
#define PK_LAUNCH_CHECK(name)                                                        \
  do {                                                                               \
    hipError_t pk_e_ = hipGetLastError();                                            \
    if (pk_e_ != hipSuccess) {                                                       \
      ::pk::set_error("%s: launch failed: %s", name, hipGetErrorString(pk_e_));       \
      return PK_ERR_LAUNCH;                                                          \
    }                                                                                \
  } while (0)

inline bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
inline bool aligned4(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 3u) == 0; }

// Per-device GELU table: 65536 bf16 entries indexed by the bf16 input bits,
// built on the device on first use.  Returns its device address for the
// current device (kernels take it as an argument).
int gelu_table(const uint16_t **table);
// Library-owned per-device scratch for entry points without a workspace arg.
int library_workspace(size_t bytes, void **ptr);

// ---- device helpers ------------------------------------------------------
__device__ __forceinline__ float bf2f(uint32_t b) { return __uint_as_float(b << 16); }

__device__ __forceinline__ uint32_t f2bf(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7F800000u) == 0x7F800000u && (u & 0x007FFFFFu) != 0u) return (u >> 16) | 0x0040u;
  u += 0x7FFFu + ((u >> 16) & 1u);
  return u >> 16;
}

// Two bf16 in one dword: low half = element 0.
__device__ __forceinline__ float lo_bf(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float hi_bf(uint32_t w) { return __uint_as_float(w & 0xFFFF0000u); }
__device__ __forceinline__ uint32_t pack_bf(float a, float b) { return f2bf(a) | (f2bf(b) << 16); }

template <typename T>
__device__ __forceinline__ T wave_sum(T v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}

}  // namespace pk
