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
#include "workspace.hpp"

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

// ---------------------------------------------------------------------------
// x / d for the elements of one row (d > 0 the row's RMS; the RMSNorm kernels
// of rowwise.hip), bit for bit the
// IEEE division: with y = RN(1/d), q = RN(x y), e = fma(-q, d, x) is exact and
// fma(e, y, q) is the correctly rounded quotient (Markstein's theorem) when no
// step underflows or overflows, which d in [2^-30, 2^30] and |x| in
// [2^-64, 2^64] guarantee.  A wave whose elements all qualify takes three
// operations per element instead of the ~10 of the division sequence;
// otherwise the wave divides every element.  Checked against IEEE
// division for all 65536 bf16 numerators x 2000 divisors on the CPU
// (tests/cpp/row_division_check.c; 20000 divisors in a longer run, no
// mismatch) and x 4096 divisors on the device (pk_check_row_division).
// ---------------------------------------------------------------------------
__device__ __forceinline__ bool div_row_ok(float d) { return d >= 0x1p-30f && d <= 0x1p30f; }
__device__ __forceinline__ bool div_elem_ok(float x) {
  const float a = fabsf(x);
  return a >= 0x1p-64f && a <= 0x1p64f;
}
__device__ __forceinline__ float div_fast(float x, float d, float y) {
  const float q = x * y;
  return fmaf(fmaf(-q, d, x), y, q);
}
// The element test on bf16 numerators held two per 32-bit word, at 1.5
// operations per element: bf16 magnitudes (bits & 0x7FFF) order like unsigned
// integers, and |x| in [2^-64, 2^64) is exactly magnitude bits in [0x1F80,
// 0x5F80) (zero of either sign falls outside).  DivSpan keeps the running
// minimum and maximum magnitude of both halves with packed 16-bit integer
// min / max; div_span_ok tests the span once.
typedef unsigned short pk_u16x2 __attribute__((ext_vector_type(2)));
struct DivSpan {
  pk_u16x2 lo = {0xFFFF, 0xFFFF}, hi = {0, 0};
};
__device__ __forceinline__ void div_span_add(DivSpan &sp, uint32_t two_bf16) {
  const pk_u16x2 m = __builtin_bit_cast(pk_u16x2, two_bf16 & 0x7FFF7FFFu);
  sp.lo = __builtin_elementwise_min(sp.lo, m);
  sp.hi = __builtin_elementwise_max(sp.hi, m);
}
__device__ __forceinline__ bool div_span_ok(const DivSpan &sp) {
  return (sp.lo.x < sp.lo.y ? sp.lo.x : sp.lo.y) >= 0x1F80 && (sp.hi.x > sp.hi.y ? sp.hi.x : sp.hi.y) < 0x5F80;
}

// Per-device compact GELU table (see gelu_bits), built on the device on first
// use.  Returns its device address for the current device (kernels take it as
// an argument).
int gelu_table(const uint16_t **table);
// Device address (current device) of the static split-K scratch of
// launch_matmul_int8_noalloc; looked up once per device.  `out` may be null.
int int8_scratch_setup(void **out);

// Configurations in the tuning-cache vocabulary (each defined beside the
// dispatcher it describes).  *_configs write min(total, cap) entries and
// return the total; the bool functions describe the built-in choice.
int gemm_configs(int M, int N, int K, pk_config *out, int cap);
bool gemm_default(int M, int N, int K, pk_config *out);
int int8_configs(int M, int N, int K, pk_config *out, int cap);
bool int8_default(int M, int N, int K, pk_config *out);
bool rmsnorm_matmul_config(int M, int N, int K, pk_config *out);
bool rmsnorm_config(int rows, int cols, pk_config *out);
bool softmax_config(int rows, int cols, pk_config *out);
int rmsnorm_configs(int rows, int cols, pk_config *out, int cap);
int softmax_configs(int rows, int cols, pk_config *out, int cap);
int attention_configs(int S_q, int S_kv, int D, pk_config *out, int cap);
bool attention_config(int S_q, int S_kv, int D, pk_config *out);

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
//   otherwise a table value.
// Table layout (2768 entries, 5.4 KiB, computed on the device with the
// reference formula): slots [0, SPAN) hold codes 0x3B4B..0x40B1 (the
// positive ones above 0x4031 map to themselves), slot SPAN the sentinel
// 0xFFFF; slots [HALF, HALF + SPAN) hold -(0x3B4B..0x40B1) and slot
// HALF + SPAN the sentinel 0x8000.  Both signs share one index range, and a
// clamped index lands on the sentinel, whose unsigned 16-bit min with the
// input is the "above the table" result (x, or -0): see gelu_pair_common.
constexpr uint32_t GELU_TLO = 0x3B4Bu, GELU_PHI = 0x4031u, GELU_NHI = 0x40B1u;
constexpr int GELU_SPAN = (int)(GELU_NHI - GELU_TLO + 1);
constexpr int GELU_HALF = GELU_SPAN + 1;
constexpr int GELU_TABLE_SIZE = 2 * GELU_HALF;

// The bf16 code of table slot i; a sentinel slot is reported through *sentinel
// with its stored value as the result.
__device__ __forceinline__ uint32_t gelu_table_code(int i, bool *sentinel) {
  const bool neg = i >= GELU_HALF;
  const int j = neg ? i - GELU_HALF : i;
  *sentinel = j == GELU_SPAN;
  if (*sentinel) return neg ? 0x8000u : 0xFFFFu;
  return (neg ? 0x8000u : 0u) | (GELU_TLO + (uint32_t)j);
}

// Branch-free: the table is read at a clamped index for every input (always
// in bounds) and the rules are selects, so a wave never splits on the input.
__device__ __forceinline__ uint32_t gelu_bits(uint32_t u, const uint16_t *__restrict__ tab) {
  const uint32_t mag = u & 0x7FFFu;
  const bool neg = (u & 0x8000u) != 0u;
  const uint32_t off = mag - GELU_TLO;  // wraps for mag < TLO
  const bool in_tab = off < (uint32_t)GELU_SPAN;
  const uint32_t idx = in_tab ? (neg ? (uint32_t)GELU_HALF : 0u) + off : 0u;
  const uint32_t tv = tab[idx];
  const uint32_t half = f2bf(0.5f * bf2f(u));
  uint32_t r = neg ? 0x8000u : u;        // |x| above the table: x or -0
  r = mag < GELU_TLO ? half : r;         // |x| below the table: 0.5 x
  r = u == 0xFF80u ? 0xFFC0u : r;        // -inf
  r = mag > 0x7F80u ? (u | 0x0040u) : r; // NaN -> quiet NaN
  return in_tab ? tv : r;
}

// Two GELU codes per register (low half = element 0), with 16-bit packed
// integer ops, for the common case: neither code is a NaN or an infinity and
// each magnitude is 0 or >= 0x0100 (exponent field >= 2).  Same results as
// gelu_bits there:
//   mag < TLO      -> bf16(0.5 x) = x with the exponent field lowered by one
//                     (exact for exponent fields >= 2), or the zero itself
//   table range    -> tab[(neg ? HALF : 0) + mag - TLO]
//   above it       -> the index clamps to the sentinel (0xFFFF positive,
//                     0x8000 negative) and min(sentinel, x) is x or -0
// Every table value v satisfies v <= x as unsigned 16-bit codes (|GELU(x)| <=
// |x| with the sign of x, or +0), so min(tab[idx], x) is the table value
// inside the range as well.  15-bit magnitudes make "a < b" the sign bit of
// the packed difference; every lookup is in bounds; the select is one
// bit-field insert of both halves.
typedef unsigned short pk_u16x2 __attribute__((ext_vector_type(2)));
typedef short pk_i16x2 __attribute__((ext_vector_type(2)));

// The packed operations of gelu_pair_common as instructions: written as
// vector-of-u16 C, the compiler turns the min/sub and arithmetic-shift masks
// into per-half compares and selects; pinned, each is one instruction for both
// halves (given the magnitudes, the pair takes 9 packed instructions, two LDS
// reads and their two address computations, and one combine).  Inline
// constants of packed ops fill only the low half, so op_sel_hi selects the low
// half for both lanes.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ uint32_t pk_vsub_u16(uint32_t a, uint32_t b) {
  uint32_t r;
  asm("v_pk_sub_u16 %0, %1, %2" : "=v"(r) : "v"(a), "s"(b));
  return r;
}
__device__ __forceinline__ uint32_t pk_vmin_u16(uint32_t a, uint32_t b) {
  uint32_t r;
  asm("v_pk_min_u16 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
  return r;
}
__device__ __forceinline__ uint32_t pk_vmin_u16s(uint32_t a, uint32_t b) {
  uint32_t r;
  asm("v_pk_min_u16 %0, %1, %2" : "=v"(r) : "v"(a), "s"(b));
  return r;
}
__device__ __forceinline__ uint32_t pk_vasr15_i16(uint32_t a) {
  uint32_t r;
  asm("v_pk_ashrrev_i16 %0, 15, %1 op_sel_hi:[0,1]" : "=v"(r) : "v"(a));
  return r;
}
__device__ __forceinline__ uint32_t pk_vbfi(uint32_t m, uint32_t a, uint32_t b) {
  uint32_t r;
  asm("v_bfi_b32 %0, %1, %2, %3" : "=v"(r) : "v"(m), "v"(a), "v"(b));
  return r;
}
__device__ __forceinline__ uint32_t pk_vbfi_s(uint32_t m, uint32_t a, uint32_t b) {
  uint32_t r;
  asm("v_bfi_b32 %0, %1, %2, %3" : "=v"(r) : "s"(m), "v"(a), "v"(b));
  return r;
}
__device__ __forceinline__ uint32_t pk_vlshr15_u16(uint32_t a) {
  uint32_t r;
  asm("v_pk_lshrrev_b16 %0, 15, %1 op_sel_hi:[0,1]" : "=v"(r) : "v"(a));
  return r;
}
__device__ __forceinline__ uint32_t pk_vmad_u16s(uint32_t a, uint32_t b, uint32_t c) {
  uint32_t r;
  asm("v_pk_mad_u16 %0, %1, %2, %3" : "=v"(r) : "v"(a), "s"(b), "v"(c));
  return r;
}
__device__ __forceinline__ uint32_t pk_vsubsat_u16(uint32_t a, uint32_t b) {
  uint32_t r;
  asm("v_pk_sub_u16 %0, %1, %2 clamp" : "=v"(r) : "v"(a), "s"(b));
  return r;
}
__device__ __forceinline__ uint32_t pk_vmax_u16(uint32_t a, uint32_t b) {
  uint32_t r;
  asm("v_pk_max_u16 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
  return r;
}
#pragma clang diagnostic pop
// Nonzero when either code of the pair leaves gelu_pair_common's domain: a
// NaN or an infinity (magnitude >= 0x7F80) or a nonzero magnitude below
// 0x0100 (exponent field 0 or 1).  Per half, mag + c sets bit 15 exactly when
// mag >= 0x8000 - c, and no sum carries into the next half (mag <= 0x7FFF).
__device__ __forceinline__ uint32_t gelu_pair_special(uint32_t w) {
  const uint32_t mag = w & 0x7FFF7FFFu;
  const uint32_t nonzero = mag + 0x7FFF7FFFu;  // mag >= 1
  const uint32_t normal = mag + 0x7F007F00u;   // mag >= 0x0100
  const uint32_t inf_nan = mag + 0x00800080u;  // mag >= 0x7F80
  return ((nonzero & ~normal) | inf_nan) & 0x80008000u;
}

// The domain test of gelu_pair_special accumulated over many pairs with two
// packed min/max instructions per pair: mn keeps the least (mag - 1) per half
// (a zero magnitude wraps to 0xFFFF), mx the greatest magnitude.  Some code
// left the domain exactly when a nonzero magnitude was below 0x0100
// (mag - 1 < 0x00FF) or a magnitude reached 0x7F80.
struct GeluVote {
  uint32_t mn, mx;
};
__device__ __forceinline__ GeluVote gelu_vote_init() { return {0xFFFFFFFFu, 0u}; }
// mag = w & 0x7FFF7FFF of the pair w.
__device__ __forceinline__ void gelu_vote_add(GeluVote &v, uint32_t mag) {
  v.mn = pk_vmin_u16(v.mn, pk_vsub_u16(mag, 0x00010001u));
  v.mx = pk_vmax_u16(v.mx, mag);
}
__device__ __forceinline__ bool gelu_vote_special(const GeluVote &v) {
  const uint32_t mn = min(v.mn & 0xFFFFu, v.mn >> 16), mx = max(v.mx & 0xFFFFu, v.mx >> 16);
  return mn < 0x00FFu || mx >= 0x7F80u;
}

// gelu_pair_common in two steps, so that a caller can issue the table reads of
// many pairs before it needs any of them: the table index of both codes (and
// the offsets mag - TLO, whose sign bit marks |x| < TLO), then the result from
// the two table values.  mag = w & 0x7FFF7FFF is shared with gelu_vote_add.
struct GeluPairIdx {
  uint32_t off, idx;
};
__device__ __forceinline__ GeluPairIdx gelu_pair_index(uint32_t w, uint32_t mag) {
  constexpr uint32_t TLO2 = GELU_TLO | (GELU_TLO << 16);
  constexpr uint32_t CLAMP2 = (uint32_t)GELU_SPAN | ((uint32_t)GELU_SPAN << 16);  // sentinel slot
  constexpr uint32_t HALF2 = (uint32_t)GELU_HALF | ((uint32_t)GELU_HALF << 16);
  const uint32_t off = pk_vsub_u16(mag, TLO2);
  // (sign bit) * HALF + min(off, SPAN): at most 2 * SPAN + 1 < 65536
  return {off, pk_vmad_u16s(pk_vlshr15_u16(w), HALF2, pk_vmin_u16s(off, CLAMP2))};
}
__device__ __forceinline__ uint32_t gelu_pair_finish(uint32_t w, uint32_t mag, uint32_t off, uint32_t tv) {
  const uint32_t r = pk_vmin_u16(tv, w);                 // table value, or x / -0 above it
  // exponent field - 1: the magnitude less 0x80, saturating at 0, with the sign of x
  const uint32_t half = pk_vbfi_s(0x7FFF7FFFu, pk_vsubsat_u16(mag, 0x00800080u), w);
  const uint32_t m_small = pk_vasr15_i16(off);           // 0xFFFF where |x| < TLO
  return pk_vbfi(m_small, half, r);
}
__device__ __forceinline__ uint32_t gelu_pair_common(uint32_t w, const uint16_t *__restrict__ tab) {
  const uint32_t mag = w & 0x7FFF7FFFu;
  const GeluPairIdx t = gelu_pair_index(w, mag);
  const uint32_t tv = (uint32_t)tab[t.idx & 0xFFFFu] | ((uint32_t)tab[t.idx >> 16] << 16);
  return gelu_pair_finish(w, mag, t.off, tv);
}

// Both codes of a pair through the exact per-element rules.
__device__ __forceinline__ uint32_t gelu_pair_exact(uint32_t w, const uint16_t *__restrict__ tab) {
  return gelu_bits(w & 0xFFFFu, tab) | (gelu_bits(w >> 16, tab) << 16);
}

// ---- direct-to-LDS loads ----------------------------------------------------
typedef __attribute__((address_space(3))) void lds_void;

// s_waitcnt immediate (gfx9 encoding): vmcnt in bits [3:0] and [15:14],
// expcnt [6:4], lgkmcnt [11:8]; expcnt and lgkmcnt left at "no wait".
constexpr int waitcnt_vm(int n) { return (n & 0xF) | ((n >> 4) << 14) | 0x0F70; }
// lgkmcnt(0), vmcnt and expcnt left at "no wait".
constexpr int WAITCNT_LGKM0 = 0xC07F;

// Buffer resource over [base, base + bytes): loads at offsets >= bytes return 0.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)bytes, 0x00020000);
}

// The same resource as four words for inline asm: base address, stride 0,
// num_records, raw-dword access flags.  The arguments must be wave-uniform;
// readfirstlane makes that visible to the compiler so the words live in SGPRs.
typedef uint32_t pk_u32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ pk_u32x4 rsrc_words(const void *base, uint32_t bytes) {
  const uint64_t p = reinterpret_cast<uint64_t>(base);
  return pk_u32x4{(uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)p),
                  (uint32_t)__builtin_amdgcn_readfirstlane((int)((uint32_t)(p >> 32) & 0xFFFFu)),
                  (uint32_t)__builtin_amdgcn_readfirstlane((int)bytes), 0x00020000u};
}

// buffer_load_dwordx4 ... lds: lane i copies 16 bytes from rsrc + voff + soff
// to LDS address lds + 16 * i.  Issued as inline asm so that the compiler's
// wait-count pass does not track it: at loop headers that pass merges its
// per-array record of pending LDS DMA into "any array" and then waits for
// every pending load before the next LDS read, draining a ring each
// iteration.  Callers order these loads with vm_wait<N>() themselves.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
// NT: the data is read once (streamed weights), so the load is non-temporal and
// does not allocate in the caches.
template <bool NT = false>
__device__ __forceinline__ void dma_lds16(pk_u32x4 rsrc, const void *lds, uint32_t voff, uint32_t soff) {
  // lds, soff and rsrc are wave-uniform; readfirstlane keeps them in SGPRs
  // (the "s" constraint does not move a VGPR value by itself)
  const int m0 = __builtin_amdgcn_readfirstlane((int)(uint32_t)reinterpret_cast<uintptr_t>((lds_void *)lds));
  const int so = __builtin_amdgcn_readfirstlane((int)soff);
  const pk_u32x4 rs = {(uint32_t)__builtin_amdgcn_readfirstlane((int)rsrc[0]),
                       (uint32_t)__builtin_amdgcn_readfirstlane((int)rsrc[1]),
                       (uint32_t)__builtin_amdgcn_readfirstlane((int)rsrc[2]),
                       (uint32_t)__builtin_amdgcn_readfirstlane((int)rsrc[3])};
  if constexpr (NT)
    asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, %3 offen nt lds"
                 :
                 : "s"(m0), "v"(voff), "s"(rs), "s"(so)
                 : "memory", "m0");
  else
    asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
                 :
                 : "s"(m0), "v"(voff), "s"(rs), "s"(so)
                 : "memory", "m0");
}
#pragma clang diagnostic pop

// Wait until at most N of this wave's vector-memory loads are outstanding
// (loads complete in issue order); a compiler memory barrier as well.
template <int N>
__device__ __forceinline__ void vm_wait() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
__device__ __forceinline__ void lgkm_wait0() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

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

// In every lane l, the values of lanes l % 32 and l % 32 + 32 (lo, hi), from
// one v_permlane32_swap_b32 (that lane layout was checked on the device)
// instead of an LDS permute.  xor32_max / xor32_sum combine a value with the
// one of lane l ^ 32; max and + are commutative, so the result is the same
// as fmaxf(v, shfl_xor(v, 32)) / v + shfl_xor(v, 32) and equal in both lanes.
__device__ __forceinline__ void xor32_pair(float v, float &lo, float &hi) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  lo = __uint_as_float(r[0]);
  hi = __uint_as_float(r[1]);
}
__device__ __forceinline__ float xor32_max(float v) {
  float lo, hi;
  xor32_pair(v, lo, hi);
  return fmaxf(lo, hi);
}
__device__ __forceinline__ float xor32_sum(float v) {
  float lo, hi;
  xor32_pair(v, lo, hi);
  return lo + hi;
}

}  // namespace pk
