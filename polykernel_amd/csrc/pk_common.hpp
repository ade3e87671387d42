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

// Per-device compact GELU table (see gelu_bits), built on the device on first
// use.  Returns its device address for the current device (kernels take it as
// an argument).
int gelu_table(const uint16_t **table);
// Library-owned per-device scratch for entry points without a workspace arg.
int library_workspace(size_t bytes, void **ptr);

// ---- device helpers ------------------------------------------------------
__device__ __forceinline__ float bf2f(uint32_t b) { return __uint_as_float(b << 16); }

// fp32 -> bf16 bits with round-to-nearest-even and NaN -> quiet NaN
// (kernels/cpu/cpu_reference.h:52-61).  gfx950's v_cvt_pk_bf16_f32 computes
// exactly that for every one of the 2^32 inputs (NaN payloads included);
// pk_check_bf16_conversion() re-verifies it on the device.
__device__ __forceinline__ uint32_t f2bf(float f) {
  return (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)f);
}

// The reference formula itself (used only by the self-check).
__device__ __forceinline__ uint32_t f2bf_formula(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7F800000u) == 0x7F800000u && (u & 0x007FFFFFu) != 0u) return (u >> 16) | 0x0040u;
  u += 0x7FFFu + ((u >> 16) & 1u);
  return u >> 16;
}

// Two bf16 in one dword: low half = element 0.
__device__ __forceinline__ float lo_bf(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float hi_bf(uint32_t w) { return __uint_as_float(w & 0xFFFF0000u); }
typedef float pk_f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 pk_bf16x2 __attribute__((ext_vector_type(2)));
// Two fp32 -> packed bf16 (low half = a) in one v_cvt_pk_bf16_f32.
__device__ __forceinline__ uint32_t pack_bf(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((pk_f32x2){a, b}, pk_bf16x2));
}

// ---- exact GELU on bf16 codes -------------------------------------------
// kernels/cpu/cpu_reference.cpp:46-55 evaluated on a bf16 input u gives, for
// every one of the 65536 codes (checked exhaustively against the CPU oracle):
//   NaN -> quiet NaN (u | 0x40); -inf -> 0xFFC0 (the x86 default NaN);
//   |x| < bf16 0x3B4B (~0.0031): bf16(0.5 * x)  (erf's contribution is below
//       half an ulp);
//   x > 0x4031 (~2.77): x;  x < -bf16 0x40B1 (~-5.53): -0;
//   otherwise a table value: codes 0x3B4B..0x4031 and -(0x3B4B..0x40B1),
//   2638 entries (5 KiB, L1-resident) computed on the device with the
//   reference formula.
constexpr uint32_t GELU_TLO = 0x3B4Bu, GELU_PHI = 0x4031u, GELU_NHI = 0x40B1u;
constexpr int GELU_NPOS = (int)(GELU_PHI - GELU_TLO + 1);
constexpr int GELU_NNEG = (int)(GELU_NHI - GELU_TLO + 1);
constexpr int GELU_TABLE_SIZE = GELU_NPOS + GELU_NNEG;

__device__ __forceinline__ uint32_t gelu_table_code(int i) {
  return i < GELU_NPOS ? GELU_TLO + (uint32_t)i : 0x8000u | (GELU_TLO + (uint32_t)(i - GELU_NPOS));
}

__device__ __forceinline__ uint32_t gelu_bits(uint32_t u, const uint16_t *__restrict__ tab) {
  const uint32_t mag = u & 0x7FFFu;
  const bool neg = (u & 0x8000u) != 0u;
  const uint32_t hi = neg ? GELU_NHI : GELU_PHI;
  if (mag >= GELU_TLO && mag <= hi) return tab[(neg ? GELU_NPOS : 0) + (int)(mag - GELU_TLO)];
  if (mag > 0x7F80u) return u | 0x0040u;
  if (u == 0xFF80u) return 0xFFC0u;
  if (mag < GELU_TLO) return f2bf(0.5f * bf2f(u));
  return neg ? 0x8000u : u;
}

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
