// int8_stream.hpp -- the streaming int8 weight-only kernel (decode shapes),
// shared by the library (int8.hip) and by code objects emitted for tuned
// configurations (csrc/runtime/codegen.cpp): both instantiate stream_body and
// reduce8_body from this one source.
#pragma once

#include <type_traits>

#include "int8_args.h"
#include "pk_common.hpp"

namespace pk {

enum Int8Epi : int { I8_NONE = 0, I8_GELU = 1, I8_RESID = 2 };

namespace i8s {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) i16x4 lds_i16x4;
typedef int v2i32 __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) v2i32 lds_v2i32;


// Epilogue of 8 consecutive outputs from their fp32 dot products v0, v1 and
// the matching scales sc0, sc1 (and residual words rv): scale, bf16, then GELU
// or residual add, one 16-byte store to `out`.
template <int EPI>
__device__ __forceinline__ void int8_finish8(const f32x4 v0, const f32x4 v1, const f32x4 sc0, const f32x4 sc1,
                                             const u32x4 rv, const uint16_t *gelu_tab, uint16_t *out) {
  float y[8];
  {
#pragma clang fp contract(off)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      y[e] = v0[e] * sc0[e];
      y[4 + e] = v1[e] * sc1[e];
    }
  }
  uint32_t o[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    uint32_t t0 = f2bf(y[2 * e]), t1 = f2bf(y[2 * e + 1]);
    if constexpr (EPI == I8_GELU) {
      t0 = gelu_bits(t0, gelu_tab);
      t1 = gelu_bits(t1, gelu_tab);
    } else if constexpr (EPI == I8_RESID) {
      t0 = f2bf(bf2f(t0) + lo_bf(rv[e]));
      t1 = f2bf(bf2f(t1) + hi_bf(rv[e]));
    }
    o[e] = t0 | (t1 << 16);
  }
  *reinterpret_cast<u32x4 *>(out) = u32x4{o[0], o[1], o[2], o[3]};
}

// The same for outputs (m, n..n+7) of a [M, N] result, loading the scales and
// the residual.  Needs n % 8 == 0 and 16-byte aligned scale, C and R rows.
template <int EPI>
__device__ __forceinline__ void int8_epilogue8(const f32x4 v0, const f32x4 v1, int m, int n, int N,
                                               const float *scale, const uint16_t *R,
                                               const uint16_t *gelu_tab, uint16_t *C) {
  const f32x4 sc0 = *reinterpret_cast<const f32x4 *>(scale + n);
  const f32x4 sc1 = *reinterpret_cast<const f32x4 *>(scale + n + 4);
  u32x4 rv = {0, 0, 0, 0};
  if constexpr (EPI == I8_RESID) rv = *reinterpret_cast<const u32x4 *>(R + (size_t)m * N + n);
  int8_finish8<EPI>(v0, v1, sc0, sc1, rv, gelu_tab, C + (size_t)m * N + n);
}

// Split reduction, 8 outputs per thread, PK_I8_REDUCE_THREADS threads per
// workgroup: the partials of all splits are loaded with 16-byte loads
// (independent, so they are all in flight at once) and added in split order.
// The GELU lookups read the 5.4 KiB table from global memory, where it stays
// cached: copying it into each workgroup's LDS first (448 copies at config 5)
// made the decode chain 1.6 us slower (90.9 against 89.3 us, bit-identical).
// Needs N % 8 == 0 and 16-byte aligned buffers.
template <int EPI>
__device__ __forceinline__ void reduce8_body(const float *partial, int splits, int M, int N, const float *scale,
                                             const uint16_t *R, const uint16_t *gelu_tab, uint16_t *C) {
  const int64_t total = (int64_t)M * N;
  const int64_t groups = total / 8;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  auto sum_splits = [&](int64_t e, f32x4 &s0, f32x4 &s1) __attribute__((always_inline)) {
    const float *p = partial + e;
    s0 = *reinterpret_cast<const f32x4 *>(p);
    s1 = *reinterpret_cast<const f32x4 *>(p + 4);
#pragma unroll 8
    for (int sp = 1; sp < splits; ++sp) {
      const float *q = p + (size_t)sp * total;
      s0 += *reinterpret_cast<const f32x4 *>(q);
      s1 += *reinterpret_cast<const f32x4 *>(q + 4);
    }
  };
  for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < groups; t += stride) {
    const int64_t e = 8 * t;
    const int n = (int)(e % N);
    const f32x4 sc0 = *reinterpret_cast<const f32x4 *>(scale + n);
    const f32x4 sc1 = *reinterpret_cast<const f32x4 *>(scale + n + 4);
    u32x4 rv = {0, 0, 0, 0};
    if constexpr (EPI == I8_RESID) rv = *reinterpret_cast<const u32x4 *>(R + e);
    f32x4 s0, s1;
    sum_splits(e, s0, s1);
    int8_finish8<EPI>(s0, s1, sc0, sc1, rv, gelu_tab, C + e);
  }
}

// ---------------------------------------------------------------------------
// Streaming kernel (fast path: N % 16 == 0, K % 64 == 0, 16-byte aligned A/W).
//
// The weight matrix is cut into units of (column slice, K split); the host
// sizes them so that the number of units is close to a multiple of the CU
// count and every CU streams the same number of bytes once.  A workgroup owns
// one unit and 16*MT rows of A.  Its WAVES waves split the slice by columns
// (16*NT each) and all walk the unit's K range in step, so at any time a CU
// reads one contiguous run of WAVES*16*NT bytes per weight row: measured on
// MI355X, runs of >= 256 B stream at the contiguous-read rate (~5.6 TB/s)
// while 128 B runs reach only ~4.4 TB/s (DRAM pages shared by many CUs at
// different times).  The waves are independent: no barriers.
//
// Each wave runs a private ring of STAGES LDS stages of 64 k-rows, filled by
// buffer_load ... lds (HBM -> LDS without registers):
//   W part: [64 rows][NT chunks of 16 B] int8.  DMA lane i of instruction q
//     fills slot c = 64q + i, i.e. row c / NT, slot c % NT, which holds
//     logical chunk (c % NT) ^ xw(row): the XOR (power-of-two NT) makes the
//     8 rows of a transpose read hit distinct banks, and (NT 8 and 16) gives
//     rows 8-15 the banks rows 0-7 leave free, since the two 16-lane groups
//     of a 32-lane LDS pass read 8 rows each (45 % -> 6.5 % bank-conflict
//     cycles); odd NT needs none.
//   A part: [16*MT rows][8 chunks of 16 B] bf16 (64 k), slot s of row r holds
//     chunk s ^ (r & 7) (each wave loads its own copy from L2).
// ds_read_b64_tr_b8 turns 8 rows x 16 columns of int8 into an MFMA operand
// (lane j of a 16-lane group receives column j, rows 0..7 -- checked on the
// device); the 8 bytes are widened to bf16 exactly (v_cvt_f32_i32 with a
// sign-extending byte select, then v_cvt_pk_bf16_f32) and fed, as the first
// operand, to v_mfma_f32_16x16x32_bf16 with the activations (a ds_read_b128)
// as the second, so each lane's accumulators are 4 consecutive columns of one
// row.  Every step issues the same number of DMA loads, so each wait is a
// constant vmcnt.  Split partials are stored from those registers with
// 16-byte stores; the final epilogue (scale, bf16, GELU / residual) goes
// through the wave's own LDS region, one m-tile at a time, with 16-byte
// global accesses.
constexpr int I8S_KSTEP = 64;
// Config fields fixed by the kernel's design: int8 elements per 16-byte DMA
// lane, and 16x16x32 MFMA k-steps per 64-row ring step.
constexpr int I8S_VECTOR_WIDTH = 16, I8S_UNROLL = I8S_KSTEP / 32;

// Kernel arguments: struct pk_i8s_args of int8_args.h (host and device share it).
using I8sArgs = pk_i8s_args;

template <int NT>
__device__ __forceinline__ int i8s_xw(int row) {
  if constexpr (NT == 2) return (row >> 2) & 1;
  else if constexpr (NT == 4) return (row >> 1) & 3;
  else if constexpr (NT == 8) return (row & 7) ^ ((row >> 3) & 1);
  else if constexpr (NT == 16) return (row & 7) | ((row >> 3) & 1) << 3;
  else return 0;  // odd NT: rows already fall on distinct banks
}

__device__ __forceinline__ bf16x8 widen8(const v2i32 w) {
  const uint32_t lo = (uint32_t)w[0], hi = (uint32_t)w[1];
  const u32x4 o = {pack_bf((float)(int8_t)lo, (float)(int8_t)(lo >> 8)),
                   pack_bf((float)(int8_t)(lo >> 16), (float)(int8_t)(lo >> 24)),
                   pack_bf((float)(int8_t)hi, (float)(int8_t)(hi >> 8)),
                   pack_bf((float)(int8_t)(hi >> 16), (float)(int8_t)(hi >> 24))};
  return __builtin_bit_cast(bf16x8, o);
}

template <int NT, int MT, int WAVES, int STAGES, int EPI>
__device__ __forceinline__ void stream_body(const I8sArgs &g) {
  static_assert((NT >= 1 && NT <= 8 && NT != 6) || NT == 16, "column tiles");
  static_assert(STAGES >= 2 && STAGES <= 6, "ring depth");
  constexpr int W_BYTES = 1024 * NT;       // 64 rows x 16*NT int8
  constexpr int A_BYTES = 2048 * MT;       // 16*MT rows x 64 bf16
  constexpr int STAGE = W_BYTES + A_BYTES; // per wave
  constexpr int P = NT + 2 * MT;           // DMA instructions per step
  constexpr int WN = 16 * NT;              // columns per wave
  constexpr int NB = WAVES * WN;           // columns per workgroup
  // the epilogue buffer [16][WN + 4] fp32 reuses the wave's region of stage 0
  static_assert(16 * (WN + 4) * 4 <= STAGE, "epilogue buffer");
  __shared__ __attribute__((aligned(1024))) uint8_t R0[WAVES * STAGE], R1[WAVES * STAGE];
  __shared__ __attribute__((aligned(1024))) uint8_t R2[STAGES > 2 ? WAVES * STAGE : 16];
  __shared__ __attribute__((aligned(1024))) uint8_t R3[STAGES > 3 ? WAVES * STAGE : 16];
  __shared__ __attribute__((aligned(1024))) uint8_t R4[STAGES > 4 ? WAVES * STAGE : 16];
  __shared__ __attribute__((aligned(1024))) uint8_t R5[STAGES > 5 ? WAVES * STAGE : 16];
  auto ring = [&](auto c) __attribute__((always_inline)) -> uint8_t * {
    constexpr int st = decltype(c)::value;
    if constexpr (st == 0) return R0;
    else if constexpr (st == 1) return R1;
    else if constexpr (st == 2) return R2;
    else if constexpr (st == 3) return R3;
    else if constexpr (st == 4) return R4;
    else return R5;
  };

  const int tid = threadIdx.x, lane = tid & 63;
  const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
  // units of one XCD (workgroup b runs on XCD b % 8) are consecutive slices
  int u = blockIdx.x;
  if (g.units % 8 == 0) u = (u & 7) * (g.units >> 3) + (u >> 3);
  const int slice = u / g.splits, split = u % g.splits;
  const int n0 = slice * NB + wid * WN;  // this wave's first column
  const int m0 = blockIdx.y * 16 * MT;
  const int ksteps = g.K / I8S_KSTEP;
  const int w0 = split * g.split_steps;
  const int T = min(ksteps, w0 + g.split_steps) - w0;  // steps of this unit
  // a wave whose columns all lie past N has nothing to load or store
  const bool active = n0 < g.N;

  // ---- DMA sources.  W: base at (row 64*w0, column n0); A: rows m0.., k 64*w0.
  // Every address stays inside W and A: columns past N (last slice) and rows
  // past M (last m-tile) are clamped onto valid data, whose products only
  // reach outputs the epilogue discards.
  const int nc = active ? n0 : 0;
  const int64_t w_bytes = (int64_t)(g.K - w0 * I8S_KSTEP) * g.N - nc;
  const int64_t a_bytes = ((int64_t)(g.M - m0) * g.K - w0 * I8S_KSTEP) * 2;
  const pk_u32x4 w_rsrc = rsrc_words(g.W + (size_t)w0 * I8S_KSTEP * g.N + nc, w_bytes > 0 ? (uint32_t)w_bytes : 0u);
  const pk_u32x4 a_rsrc = rsrc_words(g.A + (size_t)m0 * g.K + w0 * I8S_KSTEP, a_bytes > 0 ? (uint32_t)a_bytes : 0u);
  uint32_t w_off[NT];
#pragma unroll
  for (int q = 0; q < NT; ++q) {
    const int c = 64 * q + lane;
    const int row = c / NT, s = c % NT;
    const int col = min(16 * (s ^ i8s_xw<NT>(row)), g.N - 16 - nc);
    w_off[q] = (uint32_t)(row * g.N + col);
  }
  uint32_t a_off[2 * MT];
#pragma unroll
  for (int q = 0; q < 2 * MT; ++q) {
    const int c = 64 * q + lane;
    const int row = c >> 3, s = c & 7;
    const int rr = min(row, g.M - 1 - m0);
    a_off[q] = (uint32_t)(rr * g.K * 2 + 16 * (s ^ (row & 7)));
  }
  auto issue = [&](auto c, int t) __attribute__((always_inline)) {
    uint8_t *base = ring(c) + wid * STAGE;
#pragma unroll
    for (int q = 0; q < NT; ++q) dma_lds16<true>(w_rsrc, base + 1024 * q, w_off[q], t * I8S_KSTEP * g.N);
#pragma unroll
    for (int q = 0; q < 2 * MT; ++q) dma_lds16(a_rsrc, base + W_BYTES + 1024 * q, a_off[q], t * I8S_KSTEP * 2);
  };

  // ---- per-lane LDS read offsets within a stage
  const int grp = lane >> 4, gi = lane & 15;
  int w_rd[2][NT];
#pragma unroll
  for (int kk = 0; kk < 2; ++kk)
#pragma unroll
    for (int j = 0; j < NT; ++j) {
      const int row = 32 * kk + 8 * grp + (gi >> 1);
      w_rd[kk][j] = row * WN + 16 * (j ^ i8s_xw<NT>(row)) + 8 * (gi & 1);
    }
  int a_rd[2][MT];
#pragma unroll
  for (int kk = 0; kk < 2; ++kk)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int row = 16 * mt + (lane & 15);
      const int chunk = 4 * kk + grp;
      a_rd[kk][mt] = W_BYTES + row * 128 + 16 * (chunk ^ (row & 7));
    }

  f32x4 acc[MT][NT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int j = 0; j < NT; ++j) acc[mt][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  auto compute = [&](auto c) __attribute__((always_inline)) {
    const uint8_t *base = ring(c) + wid * STAGE;
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      bf16x8 a[MT];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) a[mt] = *reinterpret_cast<const bf16x8 *>(base + a_rd[kk][mt]);
#pragma unroll
      for (int j = 0; j < NT; ++j) {
        const v2i32 w = __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_v2i32 *)(base + w_rd[kk][j]));
        const bf16x8 b = widen8(w);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
          acc[mt][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(b, a[mt], acc[mt][j], 0, 0, 0);
      }
    }
  };

  using S0 = std::integral_constant<int, 0>;
  using S1 = std::integral_constant<int, 1>;
  using S2 = std::integral_constant<int, 2>;
  using S3 = std::integral_constant<int, 3>;
  using S4 = std::integral_constant<int, 4>;
  using S5 = std::integral_constant<int, 5>;
  auto dispatch = [&](int st, auto &&f) __attribute__((always_inline)) {
    switch (st) {
      case 0: f(S0{}); break;
      case 1: f(S1{}); break;
      case 2: if constexpr (STAGES > 2) f(S2{}); break;
      case 3: if constexpr (STAGES > 3) f(S3{}); break;
      case 4: if constexpr (STAGES > 4) f(S4{}); break;
      default: if constexpr (STAGES > 5) f(S5{}); break;
    }
  };

  // Waves whose columns lie past N have nothing to load or store.
  if (active) {

    // ---- prologue: steps 0 .. STAGES-2 in flight
  #pragma unroll
    for (int p = 0; p < STAGES - 1; ++p)
      if (p < T) dispatch(p, [&](auto c) __attribute__((always_inline)) { issue(c, p); });

    // ---- steady state: issue step t+STAGES-1 into the stage read at step t-1,
    // wait for step t (STAGES-1 newer steps may stay in flight), compute it.
    int t = 0;
    auto steady = [&](auto c) __attribute__((always_inline)) {
      constexpr int st = decltype(c)::value;
      using Prev = std::integral_constant<int, (st + STAGES - 1) % STAGES>;
      lgkm_wait0();  // reads of the stage being refilled are done
      issue(Prev{}, t + STAGES - 1);
      vm_wait<(STAGES - 1) * P>();
      compute(c);
      ++t;
    };
    while (t + STAGES - 1 < T) {
      steady(S0{});
      if (t + STAGES - 1 >= T) break;
      steady(S1{});
      if constexpr (STAGES > 2) { if (t + STAGES - 1 >= T) break; steady(S2{}); }
      if constexpr (STAGES > 3) { if (t + STAGES - 1 >= T) break; steady(S3{}); }
      if constexpr (STAGES > 4) { if (t + STAGES - 1 >= T) break; steady(S4{}); }
      if constexpr (STAGES > 5) { if (t + STAGES - 1 >= T) break; steady(S5{}); }
    }
    // ---- tail: everything issued; drain and compute the last steps
    vm_wait<0>();
    for (; t < T; ++t) dispatch(t % STAGES, [&](auto c) __attribute__((always_inline)) { compute(c); });

    // ---- epilogue.  The product is formed transposed (the widened weights are
    // the MFMA's first operand; the same exact products in the same k order),
    // so lane l holds, per (mt, j), the 4 consecutive columns
    // 16j + 4*(l/16) .. +3 of row 16mt + l%16.  Split partials go straight to
    // memory as 16-byte stores; the final epilogue goes one m-tile at a time
    // through this wave's region of stage 0 (buf[16][WN + 4] fp32: the 16 rows
    // of a 16-byte write fall on distinct bank quads), then 8 columns per item.
    lgkm_wait0();
    if (g.splits > 1) {
  #pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const int m = m0 + 16 * mt + gi;
  #pragma unroll
        for (int j = 0; j < NT; ++j) {
          const int n = n0 + 16 * j + 4 * grp;
          if (m < g.M && n < g.N)
            *reinterpret_cast<f32x4 *>(g.partial + ((size_t)split * g.M + m) * g.N + n) = acc[mt][j];
        }
      }
    } else {
      constexpr int LD = WN + 4;
      float *buf = reinterpret_cast<float *>(R0 + wid * STAGE);
  #pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  #pragma unroll
        for (int j = 0; j < NT; ++j) *reinterpret_cast<f32x4 *>(buf + gi * LD + 16 * j + 4 * grp) = acc[mt][j];
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        constexpr int ITEMS = 16 * (WN / 8);
  #pragma unroll
        for (int it0 = 0; it0 < ITEMS; it0 += 64) {
          const int it = it0 + lane;
          if (ITEMS % 64 != 0 && it >= ITEMS) break;
          const int r = it / (WN / 8), c8 = it % (WN / 8);
          const int m = m0 + 16 * mt + r, n = n0 + 8 * c8;
          if (m >= g.M || n >= g.N) continue;
          const f32x4 v0 = *reinterpret_cast<const f32x4 *>(buf + r * LD + 8 * c8);
          const f32x4 v1 = *reinterpret_cast<const f32x4 *>(buf + r * LD + 8 * c8 + 4);
          int8_epilogue8<EPI>(v0, v1, m, n, g.N, g.scale, g.R, g.gelu_tab, g.C);
        }
      }
    }
  }

}

}  // namespace i8s
}  // namespace pk
