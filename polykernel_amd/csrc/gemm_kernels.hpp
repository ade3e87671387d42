// gemm_kernels.hpp -- the bf16 MFMA GEMM kernels for gfx950 and the
// RMSNorm -> MatMul panel kernels (bodies), shared by the library (gemm.hip,
// which wraps them as __global__ kernels) and by code objects the emitter
// instantiates at a tuned configuration (csrc/runtime/codegen.cpp).  Both
// compile this one source.
//
// C[M,N] = A[M,K] @ B[K,N] with A K-contiguous and B N-contiguous (the
// reference layouts, kernels/cpu/cpu_reference.cpp:64-78), fp32 accumulation on
// v_mfma_f32_32x32x16_bf16; epilogues with the golden per-stage bf16 rounding
// (tests/golden/golden.py:48-66, kernels/cpu/cpu_reference.cpp:92-105):
//   EPI_NONE        c = bf16(acc)
//   EPI_BIAS_GELU   c = gelu(bf16(bf16(acc) + bias[n]))      (exact GELU, gelu_bits)
//   EPI_BIAS_RESID  c = bf16(bf16(bf16(acc) + bias[n]) + R[m,n])
//   EPI_RESID       c = bf16(bf16(acc) + R[m,n])
#pragma once

#include <type_traits>

#include "gemm_args.h"
#include "pk_common.hpp"

namespace pk {

enum Epi : int { EPI_NONE = 0, EPI_BIAS_GELU = 1, EPI_BIAS_RESID = 2, EPI_RESID = 3 };

// Kernel arguments: structs pk_gemm_args and pk_panel_args of gemm_args.h
// (host and device share them).
using GemmArgs = pk_gemm_args;
using PanelArgs = pk_panel_args;

namespace gk {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) i16x4 lds_i16x4;

constexpr int BK = 64;

// 16-byte-chunk XOR for B rows, chosen so the four rows read by one 16-lane
// ds_read_b64_tr_b16 group land on distinct LDS banks.
template <int BN>
__device__ __forceinline__ int swz_b(int k) {
  if constexpr (BN >= 128) {
    constexpr int t[4] = {0, 4, 10, 14};
    return t[k & 3];
  } else {
    return (k & 3) * 2;
  }
}

// LDS: 64 banks of 4 bytes; a ds_read_b128 is served 16 lanes (256 B) at a
// time.  A operand rows of 128 B: the 16 rows one group reads span two bank
// halves by row parity, and XOR-ing the chunk with (row >> 1) & 7 spreads the 8
// rows of each parity over all 8 chunk positions (row & 7 gave only 4).
__device__ __forceinline__ int swz_a64(int row) { return (row >> 1) & 7; }

__device__ __forceinline__ bf16x8 lds_read_a(const uint16_t *p) {
  return __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4 *>(p));
}

__device__ __forceinline__ i16x4 lds_read_tr(const uint16_t *p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4 *)(p));
}

template <int EPI>
__device__ __forceinline__ uint16_t epilogue(float acc, int m, int n, const GemmArgs &g,
                                             float bias_n) {
#pragma clang fp contract(off)
  const float t = bf2f(f2bf(acc));
  if constexpr (EPI == EPI_NONE) {
    return (uint16_t)f2bf(acc);
  } else if constexpr (EPI == EPI_BIAS_GELU) {
    const uint32_t u = f2bf(t + bias_n);
    return (uint16_t)gelu_bits(u, g.gelu_tab);
  } else if constexpr (EPI == EPI_BIAS_RESID) {
    const float u = bf2f(f2bf(t + bias_n));
    return (uint16_t)f2bf(u + bf2f(g.R[(size_t)m * g.N + n]));
  } else {
    return (uint16_t)f2bf(t + bf2f(g.R[(size_t)m * g.N + n]));
  }
}

// One 32x32 accumulator block of this lane: element i is row mb + (i/4)*8 + i%4
// of column n.  All epilogue loads (GELU table, residual) are issued before
// any store so they overlap instead of serialising load -> store pairs.
template <int EPI>
__device__ __forceinline__ void store_block(const f32x16 &acc, int mb, int n, bool nok,
                                            const GemmArgs &g, float bias_n) {
  uint16_t v[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int m = mb + (i >> 2) * 8 + (i & 3);
    const int mc = min(m, g.M - 1);
    v[i] = epilogue<EPI>(acc[i], mc, nok ? n : 0, g, bias_n);
  }
  if (!nok) return;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int m = mb + (i >> 2) * 8 + (i & 3);
    if (m < g.M) g.C[(size_t)m * g.N + n] = v[i];
  }
}

// Map the linear block id to (tile_m, tile_n): contiguous per-XCD bands
// (blocks are dispatched round-robin over the 8 XCDs), then grouped raster.
__device__ __forceinline__ void tile_coords(int bid, int tm, int tn, int &mt, int &nt) {
  const int total = tm * tn;
  int b = bid;
  if ((total & 7) == 0) b = (bid & 7) * (total >> 3) + (bid >> 3);
  constexpr int GM = 8;
  const int group = b / (GM * tn);
  const int first_m = group * GM;
  const int gsize = min(tm - first_m, GM);
  const int in_group = b - group * GM * tn;
  mt = first_m + in_group % gsize;
  nt = in_group / gsize;
}

// ---------------------------------------------------------------------------
// Main GEMM kernel.  ALIGNED: K % 8 == 0, N % 8 == 0 and 16-byte aligned A/B,
// so every 16-byte chunk is entirely in or out of bounds.
// ---------------------------------------------------------------------------
template <int BM, int BN, int WM, int WN, int EPI, bool ALIGNED>
__device__ __forceinline__ void gemm_reg_body(GemmArgs g) {
  constexpr int NT = WM * WN * 64;
  constexpr int TM = BM / WM, TN = BN / WN;
  constexpr int FM = TM / 32, FN = TN / 32;
  constexpr int A_CHUNKS = BM * BK / 8, B_CHUNKS = BK * BN / 8;
  constexpr int AC = A_CHUNKS / NT, BC = B_CHUNKS / NT;
  static_assert(A_CHUNKS % NT == 0 && B_CHUNKS % NT == 0, "tile/thread mismatch");
  static_assert(FM >= 1 && FN >= 1, "sub-tile smaller than one MFMA block");
  constexpr int BROW_CHUNKS = BN / 8;

  __shared__ __attribute__((aligned(16))) uint16_t As[2][BM * BK];
  __shared__ __attribute__((aligned(16))) uint16_t Bs[2][BK * BN];

  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int wm = wid / WN, wn = wid % WN;
  const int tm = (g.M + BM - 1) / BM, tn = (g.N + BN - 1) / BN;
  int mt, nt;
  tile_coords(blockIdx.x, tm, tn, mt, nt);
  const int m0 = mt * BM, n0 = nt * BN;
  const int KT = (g.K + BK - 1) / BK;

  u32x4 ra[AC], rb[BC];

  auto load_tiles = [&](int kt) {
    const int k0 = kt * BK;
#pragma unroll
    for (int i = 0; i < AC; ++i) {
      const int q = tid + i * NT, row = q >> 3, c = q & 7;
      const int gm = m0 + row, gk = k0 + c * 8;
      if constexpr (ALIGNED) {
        ra[i] = (gm < g.M && gk < g.K)
                    ? *reinterpret_cast<const u32x4 *>(g.A + (size_t)gm * g.K + gk)
                    : u32x4{0, 0, 0, 0};
      } else {
        uint32_t w[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint32_t lo = (gm < g.M && gk + 2 * e < g.K) ? g.A[(size_t)gm * g.K + gk + 2 * e] : 0u;
          const uint32_t hi =
              (gm < g.M && gk + 2 * e + 1 < g.K) ? g.A[(size_t)gm * g.K + gk + 2 * e + 1] : 0u;
          w[e] = lo | (hi << 16);
        }
        ra[i] = u32x4{w[0], w[1], w[2], w[3]};
      }
    }
#pragma unroll
    for (int i = 0; i < BC; ++i) {
      const int q = tid + i * NT, row = q / BROW_CHUNKS, c = q % BROW_CHUNKS;
      const int gk = k0 + row, gn = n0 + c * 8;
      if constexpr (ALIGNED) {
        rb[i] = (gk < g.K && gn < g.N)
                    ? *reinterpret_cast<const u32x4 *>(g.B + (size_t)gk * g.N + gn)
                    : u32x4{0, 0, 0, 0};
      } else {
        uint32_t w[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint32_t lo = (gk < g.K && gn + 2 * e < g.N) ? g.B[(size_t)gk * g.N + gn + 2 * e] : 0u;
          const uint32_t hi =
              (gk < g.K && gn + 2 * e + 1 < g.N) ? g.B[(size_t)gk * g.N + gn + 2 * e + 1] : 0u;
          w[e] = lo | (hi << 16);
        }
        rb[i] = u32x4{w[0], w[1], w[2], w[3]};
      }
    }
  };

  auto store_tiles = [&](int s) {
#pragma unroll
    for (int i = 0; i < AC; ++i) {
      const int q = tid + i * NT, row = q >> 3, c = q & 7;
      *reinterpret_cast<u32x4 *>(&As[s][row * BK + ((c ^ swz_a64(row)) << 3)]) = ra[i];
    }
#pragma unroll
    for (int i = 0; i < BC; ++i) {
      const int q = tid + i * NT, row = q / BROW_CHUNKS, c = q % BROW_CHUNKS;
      *reinterpret_cast<u32x4 *>(&Bs[s][row * BN + ((c ^ swz_b<BN>(row)) << 3)]) = rb[i];
    }
  };

  f32x16 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

  // Per-lane LDS offsets (elements) that do not depend on the k-substep.
  const int a_row0 = wm * TM + (lane & 31);
  const int a_half = lane >> 5;
  const int grp = lane >> 4, gi = lane & 15;
  const int b_krow = 8 * (grp >> 1) + (gi >> 2);        // + 16*s + 4*r
  const int b_col0 = wn * TN + 16 * (grp & 1) + 4 * (gi & 3);  // + 32*fn

  load_tiles(0);
  store_tiles(0);
  __syncthreads();

  for (int kt = 0; kt < KT; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < KT) load_tiles(kt + 1);
    const uint16_t *as = As[cur];
    const uint16_t *bs = Bs[cur];
#pragma unroll
    for (int s = 0; s < BK / 16; ++s) {
      bf16x8 af[FM], bfr[FN];
#pragma unroll
      for (int fm = 0; fm < FM; ++fm) {
        const int row = a_row0 + fm * 32;
        const int c = 2 * s + a_half;
        af[fm] = lds_read_a(as + row * BK + ((c ^ swz_a64(row)) << 3));
      }
#pragma unroll
      for (int fn = 0; fn < FN; ++fn) {
        i16x4 h[2];
#pragma unroll
        for (int r = 0; r < 2; ++r) {
          const int k = 16 * s + 4 * r + b_krow;
          const int col = b_col0 + 32 * fn;
          const int c = col >> 3;
          h[r] = lds_read_tr(bs + k * BN + ((c ^ swz_b<BN>(k)) << 3) + (col & 7));
        }
        short tmp[8] = {h[0][0], h[0][1], h[0][2], h[0][3], h[1][0], h[1][1], h[1][2], h[1][3]};
        bfr[fn] = __builtin_bit_cast(bf16x8, tmp);
      }
#pragma unroll
      for (int fm = 0; fm < FM; ++fm)
#pragma unroll
        for (int fn = 0; fn < FN; ++fn)
          acc[fm][fn] =
              __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[fm], bfr[fn], acc[fm][fn], 0, 0, 0);
    }
    if (kt + 1 < KT) store_tiles(cur ^ 1);
    __syncthreads();
  }

  // Epilogue: acc[fm][fn][i] -> row (i/4)*8 + (lane/32)*4 + i%4, col lane%32.
#pragma unroll
  for (int fn = 0; fn < FN; ++fn) {
    const int n = n0 + wn * TN + fn * 32 + (lane & 31);
    const bool nok = n < g.N;
    float bias_n = 0.f;
    if constexpr (EPI == EPI_BIAS_GELU || EPI == EPI_BIAS_RESID)
      bias_n = (nok && g.bias) ? bf2f(g.bias[n]) : 0.f;
#pragma unroll
    for (int fm = 0; fm < FM; ++fm) {
      const int mb = m0 + wm * TM + fm * 32 + (lane >> 5) * 4;
      store_block<EPI>(acc[fm][fn], mb, n, nok, g, bias_n);
    }
  }
}

// ---------------------------------------------------------------------------
// Large-tile GEMM (the MLP block path).  256x256 per workgroup, W = 8 waves
// in a 2x4 grid (WNN = 4 along N), each wave owning a 128x64 sub-tile (8 MFMA
// accumulator blocks, 128 fp32 per lane), two waves per SIMD: while one waits
// at the barrier, on its LDS reads or on issuing its DMA, the other keeps the
// matrix core busy.  Other instantiations of the template: W = 4 (one wave
// per SIMD, 128x128 sub-tiles; config-2 GEMM1 474 -> 452 us and GEMM2
// 443 -> 423 us going to 8 waves) and the 4x2 grid of 64x128 sub-tiles (0.5 %
// slower than 2x4: two more LDS read instructions per substep); all
// bit-identical.  K advances in tiles of 32 through a
// STAGES-deep LDS ring (4 or 5) filled by buffer_load_dwordx4 ... lds
// (global -> LDS without VGPR staging) issued STAGES-1 tiles ahead.  Per
// k-tile and wave:
//     MFMAs of substep 0, interleaved with the fragment reads of substep 1 |
//     wait own reads and own DMA of tile t+1, s_barrier |
//     MFMAs of substep 1, interleaved with the DMA of tile t+STAGES into the
//     freed stage and the fragment reads of tile t+1 substep 0
// so the single barrier sits behind queued MFMA work and every LDS read is
// issued one substep before its use.  The DMA is issued as inline asm
// (dma_lds16) and ordered only by the explicit waits below.  Requires K % 32 == 0, N % 8 == 0 and
// 16-byte aligned A/B; out-of-range rows/columns are clamped to valid memory
// (their results are never stored).
// ---------------------------------------------------------------------------
constexpr int G2_BM = 256, G2_BN = 256, G2_BK = 32, G2_STAGES = 4;
constexpr int G2_WAVES = 8, G2_WAVES_N = 4;
constexpr int G2_THREADS = G2_WAVES * 64;

// A rows of 64 B (the DMA kernel's 32-wide k-tiles): the 16 rows of a read
// group fall 4 to each 64-byte quarter of the banks by row & 3, and
// (row >> 2) & 3 gives those 4 rows distinct chunks (conflict-free; (row >> 1)
// & 3 left 2-way conflicts).
__device__ __forceinline__ int swz_a32(int row) { return (row >> 2) & 3; }

template <int EPI, int STAGES, int W = G2_WAVES, int WNN = G2_WAVES_N>
__device__ __forceinline__ void gemm_dma_body(GemmArgs g) {
  static_assert(STAGES == 4 || STAGES == 5, "ring depth");
  static_assert(W == 4 || W == 8, "waves");
  constexpr int NTHR = W * 64;
  constexpr int WMN = W / WNN;          // waves along M (WNN along N)
  constexpr int TM = G2_BM / WMN;       // rows per wave
  constexpr int TN = G2_BN / WNN;       // columns per wave
  constexpr int FM = TM / 32;           // 32-row MFMA blocks per wave
  constexpr int FN = TN / 32;           // 32-column MFMA blocks per wave
  constexpr int NA = 16 / W, NB = 16 / W;  // 1 KiB DMA loads per wave per k-tile
  constexpr int DPT = NA + NB;
  constexpr int NU = FM + FN;           // fragment-read units per substep
  constexpr int NM = FM * FN;           // MFMAs per substep
  constexpr int NJ = 4096 / NTHR;       // 16-byte epilogue chunks per thread per half
  constexpr int A_STAGE = G2_BM * G2_BK;  // elements
  constexpr int B_STAGE = G2_BK * G2_BN;
  // One array per ring stage: distinct LDS objects let the compiler see that a
  // DMA into one stage does not alias reads of another, so it adds no waits of
  // its own; the explicit vmcnt waits below order each stage.
  __shared__ __attribute__((aligned(1024))) uint16_t As0[A_STAGE], As1[A_STAGE], As2[A_STAGE], As3[A_STAGE];
  __shared__ __attribute__((aligned(1024))) uint16_t Bs0[B_STAGE], Bs1[B_STAGE], Bs2[B_STAGE], Bs3[B_STAGE];
  __shared__ __attribute__((aligned(1024))) uint16_t As4[STAGES > 4 ? A_STAGE : 8], Bs4[STAGES > 4 ? B_STAGE : 8];
  auto a_stage = [&](auto c) -> uint16_t * {
    constexpr int st = decltype(c)::value;
    if constexpr (st == 0) return As0;
    else if constexpr (st == 1) return As1;
    else if constexpr (st == 2) return As2;
    else if constexpr (st == 3) return As3;
    else return As4;
  };
  auto b_stage = [&](auto c) -> uint16_t * {
    constexpr int st = decltype(c)::value;
    if constexpr (st == 0) return Bs0;
    else if constexpr (st == 1) return Bs1;
    else if constexpr (st == 2) return Bs2;
    else if constexpr (st == 3) return Bs3;
    else return Bs4;
  };

  const int tid = threadIdx.x, lane = tid & 63;
  // wave index as a scalar: every LDS destination (M0) below is then computed
  // in scalar registers
  const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wid / WNN, wn = wid % WNN;
  const int tm = (g.M + G2_BM - 1) / G2_BM, tn = (g.N + G2_BN - 1) / G2_BN;
  int mt, nt;
  tile_coords(blockIdx.x, tm, tn, mt, nt);
  const int m0 = mt * G2_BM, n0 = nt * G2_BN;
  const int KT = g.K / G2_BK;

  // ---- DMA sources: buffer_load ... lds with a resource descriptor per
  // operand (A: rows m0.., B: columns n0..), a loop-invariant per-lane byte
  // offset (voffset) and the per-tile advance as the scalar soffset, so the
  // issue needs no address arithmetic in vector registers.
  // A: wave w, instr j covers rows 64w + 16j + lane/4, physical chunk lane%4.
  uint32_t a_off[NA];
#pragma unroll
  for (int j = 0; j < NA; ++j) {
    const int r = (G2_BM / W) * wid + 16 * j + (lane >> 2);
    const int c = (lane & 3) ^ swz_a32(r);
    const int rr = min(r, g.M - 1 - m0);
    a_off[j] = (uint32_t)(rr * g.K + 8 * c) * 2u;
  }
  // B: wave w, instr j covers rows 8w + 2j + lane/32, physical chunk lane%32.
  uint32_t b_off[NB];
#pragma unroll
  for (int j = 0; j < NB; ++j) {
    const int r = (G2_BK / W) * wid + 2 * j + (lane >> 5);
    const int c = (lane & 31) ^ swz_b<G2_BN>(r);
    const int cc = min(8 * c, g.N - 8 - n0);
    b_off[j] = (uint32_t)(r * g.N + cc) * 2u;
  }
  // Every A offset stays inside this tile's (at most) 256 rows, so the
  // record count is that panel's size, which fits 32 bits whenever 256 * K * 2
  // does (checked by the dispatcher) -- the whole remaining matrix need not.
  const pk_u32x4 a_rsrc = rsrc_words(g.A + (size_t)m0 * g.K, (uint32_t)((size_t)min(g.M - m0, G2_BM) * g.K * 2));
  const pk_u32x4 b_rsrc = rsrc_words(g.B + n0, (uint32_t)(((size_t)g.K * g.N - n0) * 2));
  auto issue_one = [&](auto c, int t, int j) __attribute__((always_inline)) {
    if (j < NA)
      dma_lds16(a_rsrc, &a_stage(c)[((G2_BM / W) * wid + 16 * j) * G2_BK], a_off[j], t * (G2_BK * 2));
    else
      dma_lds16(b_rsrc, &b_stage(c)[((G2_BK / W) * wid + 2 * (j - NA)) * G2_BN], b_off[j - NA],
                t * (G2_BK * 2) * g.N);
  };
  auto issue = [&](auto c, int t) {
#pragma unroll
    for (int j = 0; j < DPT; ++j) issue_one(c, t, j);
  };

  // ---- per-lane fragment read offsets (elements within a stage)
  int a_rd[FM][2];
#pragma unroll
  for (int fm = 0; fm < FM; ++fm) {
    const int row = wm * TM + fm * 32 + (lane & 31);
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const int c = 2 * s + (lane >> 5);
      a_rd[fm][s] = row * G2_BK + ((c ^ swz_a32(row)) << 3);
    }
  }
  const int grp = lane >> 4, gi = lane & 15;
  int b_rd[FN][2][2];
#pragma unroll
  for (int fn = 0; fn < FN; ++fn)
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
      for (int r = 0; r < 2; ++r) {
        const int k = 16 * s + 8 * (grp >> 1) + 4 * r + (gi >> 2);
        const int col = wn * TN + fn * 32 + 16 * (grp & 1) + 4 * (gi & 3);
        const int c = col >> 3;
        b_rd[fn][s][r] = k * G2_BN + ((c ^ swz_b<G2_BN>(k)) << 3) + (col & 7);
      }

  struct Frag {
    bf16x8 a[FM];
    bf16x8 b[FN];
  };
  // Fragment reads in 8 units (u < 4: A block u; u >= 4: B block u-4, two
  // transpose reads joined without repacking) so they can be spread over the
  // MFMA stream.  (Measured: this order beats issuing them in order of first
  // use.)
  auto read_unit = [&](Frag &f, auto c, int s, int u) {
    const uint16_t *as = a_stage(c);
    const uint16_t *bs = b_stage(c);
    const int fm = u;
    if (u < FM) {
      f.a[fm] = lds_read_a(as + a_rd[fm][s]);
    } else {
      const int fn = u - FM;
      const i16x4 h0 = lds_read_tr(bs + b_rd[fn][s][0]);
      const i16x4 h1 = lds_read_tr(bs + b_rd[fn][s][1]);
      f.b[fn] = __builtin_bit_cast(bf16x8, __builtin_shufflevector(h0, h1, 0, 1, 2, 3, 4, 5, 6, 7));
    }
  };
  auto read_frag = [&](Frag &f, auto c, int s) {
#pragma unroll
    for (int u = 0; u < NU; ++u) read_unit(f, c, s, u);
  };
  f32x16 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

  // With the GELU epilogue the product is formed transposed (W fragment as the
  // MFMA's first operand): acc[fm][fn] then holds the 32 x 32 block with lane l
  // owning output row fm*32 + l%32 and, per q, the 4 consecutive columns
  // fn*32 + 8q + 4*(l/32) + (0..3), so the epilogue works on row-contiguous
  // registers without staging the tile through LDS.  Each output is the same
  // exact bf16 products summed in the same k order.
  constexpr bool TRANSPOSED = EPI == EPI_BIAS_GELU;
  auto mfma_one = [&](const Frag &f, int i) {
    if constexpr (TRANSPOSED)
      acc[i / FN][i % FN] =
          __builtin_amdgcn_mfma_f32_32x32x16_bf16(f.b[i % FN], f.a[i / FN], acc[i / FN][i % FN], 0, 0, 0);
    else
      acc[i / FN][i % FN] =
          __builtin_amdgcn_mfma_f32_32x32x16_bf16(f.a[i / FN], f.b[i % FN], acc[i / FN][i % FN], 0, 0, 0);
  };

  using S0 = std::integral_constant<int, 0>;
  using S1 = std::integral_constant<int, 1>;
  using S2 = std::integral_constant<int, 2>;
  using S3 = std::integral_constant<int, 3>;
  using S4 = std::integral_constant<int, 4>;

  // The GELU epilogue's operands are loaded before the first DMA, so their
  // latency hides behind the main loop instead of opening the epilogue: this
  // thread's words of the GELU table (copied into LDS once the ring is free)
  // and the bias of the lane's 32 columns.  Issued ahead of every DMA load,
  // they are older than all of them, so the in-order vmcnt waits below still
  // count only DMA loads behind them.
  constexpr int TAB_W = (GELU_TABLE_SIZE + 1) / 2;  // table words
  constexpr int TAB_PT = (TAB_W + NTHR - 1) / NTHR;
  uint32_t tab_pre[TRANSPOSED ? TAB_PT : 1];
  uint2 bias_pre[TRANSPOSED ? FN * 4 : 1];
  if constexpr (TRANSPOSED) {
#pragma unroll
    for (int j = 0; j < TAB_PT; ++j) {
      const int i = tid + j * NTHR;
      tab_pre[j] = i < TAB_W ? reinterpret_cast<const uint32_t *>(g.gelu_tab)[i] : 0u;
    }
#pragma unroll
    for (int fn = 0; fn < FN; ++fn)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int n = n0 + wn * TN + 4 * (lane >> 5) + fn * 32 + 8 * q;
        bias_pre[fn * 4 + q] = (g.bias && n < g.N) ? *reinterpret_cast<const uint2 *>(g.bias + n) : uint2{0u, 0u};
      }
  }

  // ---- prologue: tiles 0..STAGES-2 and the A half of tile STAGES-1 in
  // flight (indices past the end are clamped to the last tile: every k-tile
  // issues the same number of DMA loads, so each wait below is a compile-time
  // vmcnt), wait for tile 0.
  using SL = std::integral_constant<int, STAGES - 1>;
  issue(S0{}, 0);
  issue(S1{}, min(1, KT - 1));
  issue(S2{}, min(2, KT - 1));
  if constexpr (STAGES > 4) issue(S3{}, min(3, KT - 1));
#pragma unroll
  for (int j = 0; j < NA; ++j) issue_one(SL{}, min(STAGES - 1, KT - 1), j);
  vm_wait<(STAGES - 2) * DPT + NA>();
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");  // no LDS access moves above the barrier
  __builtin_amdgcn_sched_barrier(0);

  Frag f0, f1;
  read_frag(f0, S0{}, 0);
  // One k-tile on ring stage C (tile t, t % STAGES == C):
  //   16 MFMAs on substep 0, a fragment-read unit of substep 1 after every
  //   second MFMA and a B load of tile t+STAGES-1 (into the stage the last
  //   barrier released) after every fourth;
  //   wait for this wave's reads of the stage and its DMA of tile t+1, barrier;
  //   16 MFMAs on substep 1, a read unit of tile t+1's substep 0 after every
  //   second and an A load of tile t+STAGES (into the stage just released)
  //   after every fourth.
  // Spreading each tile's 8 loads over both halves of a k-tile instead of
  // one half evens out the demand on the texture unit (GEMM2 shape -3.5 %).
  // Every tile's loads still precede all loads of the next tile, so the
  // vmcnt waits count the same.
  auto body = [&](auto c, int t) {
    constexpr int st = decltype(c)::value;
    using Next = std::integral_constant<int, (st + 1) % STAGES>;
    using Prev = std::integral_constant<int, (st + STAGES - 1) % STAGES>;
    const int tp_dma = min(t + STAGES - 1, KT - 1);
#pragma unroll
    for (int i = 0; i < NM; ++i) {
      mfma_one(f0, i);
      if constexpr (W == 4) {
        if ((i & 1) == 0) read_unit(f1, c, 1, i >> 1);
      } else {
        if (i < NU) read_unit(f1, c, 1, i);
      }
      if ((i & 3) == 1) issue_one(Prev{}, tp_dma, NA + (i >> 2));
      __builtin_amdgcn_sched_barrier(0);
    }
    // this wave's reads of stage st are done and its DMA of tile t+1 landed
    // (STAGES-2 newer tiles may still be in flight); then all waves agree.
    lgkm_wait0();
    vm_wait<(STAGES - 2) * DPT>();
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");  // no LDS access moves above the barrier
    __builtin_amdgcn_sched_barrier(0);
    const int tn_dma = min(t + STAGES, KT - 1);
#pragma unroll
    for (int i = 0; i < NM; ++i) {
      mfma_one(f1, i);
      if ((i & 3) == 1) issue_one(c, tn_dma, i >> 2);
      if constexpr (W == 4) {
        if ((i & 1) == 0) read_unit(f0, Next{}, 0, i >> 1);
      } else {
        if (i < NU) read_unit(f0, Next{}, 0, i);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  for (int t = 0; t < KT; t += STAGES) {
    body(S0{}, t);
    if (t + 1 < KT) body(S1{}, t + 1);
    if (t + 2 < KT) body(S2{}, t + 2);
    if (t + 3 < KT) body(S3{}, t + 3);
    if constexpr (STAGES > 4) {
      if (t + 4 < KT) body(S4{}, t + 4);
    }
  }
  // clamped tail loads may still be landing in LDS: drain before leaving
  vm_wait<0>();

  if constexpr (TRANSPOSED) {
    // ---- bias + GELU in registers, then the tile through LDS for 16-byte
    // row stores.  Lane l holds, per (fm, fn, q), the outputs (row
    // fm*32 + l%32, columns fn*32 + 8q + 4*(l/32) .. +3) of its wave's block:
    // bf16(acc) and bias in fp32, bf16 again, the paired table GELU (one wave
    // vote per fm picks it, or the exact rules when a NaN, an infinity or a
    // tiny magnitude is present), one 8-byte LDS write per 4 columns.  The
    // 256 x 256 bf16 tile fills 8 ring arrays (32 rows of 512 B each, 16-byte
    // chunk k of row r at k ^ (r % 32), its two 8-byte halves swapped in rows
    // 16-31: a 16-lane read of one row's 16 chunks and a 32-row write both
    // cover all 64 banks once); the GELU table sits in a ninth array.
    __shared__ __attribute__((aligned(16))) uint16_t TabX[STAGES > 4 ? 8 : GELU_TABLE_SIZE + 8];
    uint16_t *tab_lds = STAGES > 4 ? As4 : TabX;
    static_assert(GELU_TABLE_SIZE <= A_STAGE, "GELU table fits in one ring array");
    auto stage_row = [&](int r) -> uint16_t * {
      uint16_t *base;
      switch (r >> 5) {
        case 0: base = As0; break;
        case 1: base = As1; break;
        case 2: base = As2; break;
        case 3: base = As3; break;
        case 4: base = Bs0; break;
        case 5: base = Bs1; break;
        case 6: base = Bs2; break;
        default: base = Bs3; break;
      }
      return base + (r & 31) * G2_BN;
    };
    __syncthreads();  // every wave is done reading the ring
#pragma unroll
    for (int j = 0; j < TAB_PT; ++j)
      if (tid + j * NTHR < TAB_W) reinterpret_cast<uint32_t *>(tab_lds)[tid + j * NTHR] = tab_pre[j];
    const int gq = lane >> 5;
    const int cw = wn * TN + 4 * gq;  // tile column of the lane's first output, + fn*32 + 8q
    float bias_f[FN][4][4];
#pragma unroll
    for (int fn = 0; fn < FN; ++fn)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint2 bw = bias_pre[fn * 4 + q];
        bias_f[fn][q][0] = lo_bf(bw.x);
        bias_f[fn][q][1] = hi_bf(bw.x);
        bias_f[fn][q][2] = lo_bf(bw.y);
        bias_f[fn][q][3] = hi_bf(bw.y);
      }
    __syncthreads();  // the table is in LDS
#pragma unroll
    for (int fm = 0; fm < FM; ++fm) {
      const int r = wm * TM + fm * 32 + (lane & 31);
      uint32_t u[FN][4][2], mg[FN][4][2];
      GeluVote vote = gelu_vote_init();
#pragma unroll
      for (int fn = 0; fn < FN; ++fn)
#pragma unroll
        for (int q = 0; q < 4; ++q)
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const uint32_t t = pack_bf(acc[fm][fn][4 * q + 2 * h], acc[fm][fn][4 * q + 2 * h + 1]);
            u[fn][q][h] = pack_bf(lo_bf(t) + bias_f[fn][q][2 * h], hi_bf(t) + bias_f[fn][q][2 * h + 1]);
            mg[fn][q][h] = u[fn][q][h] & 0x7FFF7FFFu;
            gelu_vote_add(vote, mg[fn][q][h]);
          }
      if (__builtin_amdgcn_ballot_w64(gelu_vote_special(vote)) == 0) {
        GeluPairIdx t[FN][4][2];
        uint32_t tl[FN][4][2], th[FN][4][2];
#pragma unroll
        for (int fn = 0; fn < FN; ++fn)
#pragma unroll
          for (int q = 0; q < 4; ++q)
#pragma unroll
            for (int h = 0; h < 2; ++h) {
              t[fn][q][h] = gelu_pair_index(u[fn][q][h], mg[fn][q][h]);
              tl[fn][q][h] = tab_lds[t[fn][q][h].idx & 0xFFFFu];
              th[fn][q][h] = tab_lds[t[fn][q][h].idx >> 16];
            }
#pragma unroll
        for (int fn = 0; fn < FN; ++fn)
#pragma unroll
          for (int q = 0; q < 4; ++q)
#pragma unroll
            for (int h = 0; h < 2; ++h)
              u[fn][q][h] = gelu_pair_finish(u[fn][q][h], mg[fn][q][h], t[fn][q][h].off,
                                             tl[fn][q][h] | (th[fn][q][h] << 16));
      } else {
#pragma unroll
        for (int fn = 0; fn < FN; ++fn)
#pragma unroll
          for (int q = 0; q < 4; ++q)
#pragma unroll
            for (int h = 0; h < 2; ++h) u[fn][q][h] = gelu_pair_exact(u[fn][q][h], tab_lds);
      }
      uint16_t *row = stage_row(r);
#pragma unroll
      for (int fn = 0; fn < FN; ++fn)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int k = (cw + fn * 32 + 8 * q) >> 3;
          *reinterpret_cast<uint2 *>(row + 8 * (k ^ (r & 31)) + 4 * (gq ^ ((r >> 4) & 1))) =
              uint2{u[fn][q][0], u[fn][q][1]};
        }
    }
    __syncthreads();
    uint16_t *__restrict__ Cp = g.C;
    constexpr int NC = G2_BM * (G2_BN / 8) / NTHR;  // 16-byte chunks per thread
#pragma unroll
    for (int j = 0; j < NC; ++j) {
      const int qd = tid + j * NTHR;
      const int r = qd >> 5, k = qd & 31;
      const int m = m0 + r, n = n0 + 8 * k;
      u32x4 v = *reinterpret_cast<const u32x4 *>(stage_row(r) + 8 * (k ^ (r & 31)));
      // rows 16-31 of each 32-row array hold their 8-byte halves swapped; the
      // rows this j reads, (tid >> 5) + j * NTHR / 32, all fall on one side
      static_assert(NTHR / 32 == 8 || NTHR / 32 == 16, "row step of the read-back");
      if (((j * (NTHR / 32)) >> 4) & 1) v = u32x4{v[2], v[3], v[0], v[1]};
      if (m < g.M && n < g.N) *reinterpret_cast<u32x4 *>(Cp + (size_t)m * g.N + n) = v;
    }
    return;
  }

  // ---- epilogue of the other forms, staged through the (now idle) LDS ring
  // in two halves of 128 rows: waves of row-half h write t = bf16(acc) into
  // padded rows (264 elements, so the two 32-lane row groups of a write hit
  // opposite bank halves), then all threads walk the half in 16-byte row
  // chunks, apply bias / residual with vector loads and store 16 bytes at a
  // time.
  // 8-row block b of a half lives in ring array b / 3 at row offset (b % 3) * 8.
  constexpr int EP_LD = 264;
  auto ep_block = [&](int blk) -> uint16_t * {
    switch (blk / 3) {
      case 0: return As0 + (blk % 3) * 8 * EP_LD;
      case 1: return As1 + (blk % 3) * 8 * EP_LD;
      case 2: return As2 + (blk % 3) * 8 * EP_LD;
      case 3: return As3 + (blk % 3) * 8 * EP_LD;
      case 4: return (STAGES > 4 ? As4 : Bs1) + (blk % 3) * 8 * EP_LD;
      default: return Bs0 + (blk % 3) * 8 * EP_LD;
    }
  };
  __syncthreads();  // every wave is done reading the ring
  // The bias chunk of a thread's columns is the same for every row it visits
  // (its column group is tid % 32), so it is loaded once.
  uint16_t *__restrict__ Cp = g.C;
  const uint16_t *__restrict__ Rp = g.R;
  const int c_thr = tid & 31;
  u32x4 bv = {0, 0, 0, 0};
  if constexpr (EPI == EPI_BIAS_RESID)
    if (g.bias && n0 + 8 * c_thr < g.N) bv = *reinterpret_cast<const u32x4 *>(g.bias + n0 + 8 * c_thr);
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    if (wm / (WMN / 2) == h) {
#pragma unroll
      for (int fm = 0; fm < FM; ++fm)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          uint16_t *blk = ep_block((wm % (WMN / 2)) * (TM / 8) + fm * 4 + q);
#pragma unroll
          for (int fn = 0; fn < FN; ++fn) {
            const int col = wn * TN + fn * 32 + (lane & 31);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const int r = (lane >> 5) * 4 + e;
              blk[r * EP_LD + col] = (uint16_t)f2bf(acc[fm][fn][q * 4 + e]);
            }
          }
        }
    }
    __syncthreads();
#pragma unroll 4
    for (int j = 0; j < NJ; ++j) {
      const int qd = tid + j * NTHR;
      const int r = qd >> 5, c = qd & 31;  // c == c_thr
      const int m = m0 + h * 128 + r, n = n0 + 8 * c;
      if (m < g.M && n < g.N) {
        const uint16_t *src = ep_block(r >> 3) + (r & 7) * EP_LD + 8 * c;
        const u32x4 tv = *reinterpret_cast<const u32x4 *>(src);
        u32x4 ov;
        if constexpr (EPI == EPI_NONE) {
          ov = tv;
        } else {
          u32x4 rv = {0, 0, 0, 0};
          if constexpr (EPI == EPI_BIAS_RESID || EPI == EPI_RESID)
            rv = *reinterpret_cast<const u32x4 *>(Rp + (size_t)m * g.N + n);
          {
#pragma unroll
            for (int w = 0; w < 4; ++w) {
              uint32_t o2 = 0;
#pragma unroll
              for (int hh = 0; hh < 2; ++hh) {
                const float t = hh ? hi_bf(tv[w]) : lo_bf(tv[w]);
                uint32_t o;
                if constexpr (EPI == EPI_BIAS_RESID) {
                  const float u = bf2f(f2bf(t + (hh ? hi_bf(bv[w]) : lo_bf(bv[w]))));
                  o = f2bf(u + (hh ? hi_bf(rv[w]) : lo_bf(rv[w])));
                } else {
                  o = f2bf(t + (hh ? hi_bf(rv[w]) : lo_bf(rv[w])));
                }
                o2 |= o << (16 * hh);
              }
              ov[w] = o2;
            }
          }
        }
        *reinterpret_cast<u32x4 *>(Cp + (size_t)m * g.N + n) = ov;
      }
    }
    if (h == 0) __syncthreads();  // the half is consumed before the next overwrites it
  }
}


// Latency-oriented RMSNorm -> MatMul for short rows (K <= 832, the config-1
// fragment: a few MB, cache-resident, so one memory round trip dominates).
// A workgroup of 8 waves owns 32 rows x 64 columns:
//   - load the 32 x K panel of x (and gamma) into registers, then issue the
//     whole 64-column slice of W (K x 64, 128 K bytes) as buffer_load ... lds
//     DMA into LDS, every load in flight at once (loads complete in order, so
//     x first lets the normalisation start while W still arrives: 8.50 ->
//     8.34 us per config-1 launch);
//   - 16 lanes per row reduce the sum of squares (shuffles), normalise
//     x / rms * gamma exactly as the reference and store the bf16 panel in LDS
//     while W is still arriving;
//   - wave w computes column block w & 1 over K quarter w >> 1 (MFMA
//     32x32x16), the quarters are added in LDS in order and the tile is
//     stored 16 bytes at a time.
// With one wave per SIMD (4 waves, K halves) each wave normalised 96 elements
// of x and ran a 24-deep chain of dependent MFMAs; 8 waves halve both:
// config 1 7.83 -> 6.67 us per launch in a replayed graph (every output within
// the same error model; 99.07 % bit-exact to the oracle either way).
constexpr int RQ_BM = 32, RQ_BN = 64, RQ_THREADS = PK_PANEL_THREADS;
constexpr int RQ_MAX_K = 832;  // panel 64 K bytes + W slice 128 K bytes <= 160 KiB
constexpr int RQ_TPR = RQ_THREADS / RQ_BM;         // threads per x row (16)
constexpr int RQ_XPT = (RQ_MAX_K / 8 + RQ_TPR - 1) / RQ_TPR;  // x chunks (16 B) per thread at most
constexpr int RQ_KP = RQ_THREADS / 64 / 2;         // K parts (waves per column block)

__device__ __forceinline__ void rmsnorm_panel_fast_body(const PanelArgs &a) {
#pragma clang fp contract(off)
  const uint16_t *__restrict__ X = a.X;
  const uint16_t *__restrict__ gamma = a.gamma;
  const uint16_t *__restrict__ B = a.B;
  uint16_t *__restrict__ C = a.C;
  const int M = a.M, N = a.N, K = a.K;
  const float inv_cols = a.inv_cols, eps = a.eps;
  extern __shared__ __attribute__((aligned(1024))) uint8_t smem8[];
  uint16_t *Bs = reinterpret_cast<uint16_t *>(smem8);                // [K][64], chunk-swizzled
  uint16_t *Ap = reinterpret_cast<uint16_t *>(smem8 + (size_t)K * 128);  // [32][K], chunk-swizzled

  const int tid = threadIdx.x, lane = tid & 63;
  const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int tn = (N + RQ_BN - 1) / RQ_BN;
  const int mt = blockIdx.x / tn, nt = blockIdx.x % tn;
  const int m0 = mt * RQ_BM, n0 = nt * RQ_BN;
  const int kchunks = K >> 3;

  // ---- x panel -> registers: thread t owns row t / 16, chunks (t % 16) + 16 j
  const int r = tid / RQ_TPR, c0 = tid % RQ_TPR;
  const int gm = m0 + r;
  const int nxc = (kchunks - c0 + RQ_TPR - 1) / RQ_TPR;
  u32x4 xv[RQ_XPT], gv[RQ_XPT];
#pragma unroll
  for (int j = 0; j < RQ_XPT; ++j) {
    xv[j] = u32x4{0, 0, 0, 0};
    gv[j] = u32x4{0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u};  // bf16 1.0 (no gamma)
    if (j < nxc) {
      const int c = c0 + RQ_TPR * j;
      if (gm < M) xv[j] = *reinterpret_cast<const u32x4 *>(X + (size_t)gm * K + c * 8);
      if (gamma) gv[j] = *reinterpret_cast<const u32x4 *>(gamma + c * 8);
    }
  }
  // ---- W slice -> LDS: instruction q covers rows 8q..8q+7 (8 chunks each);
  // lane i fills row 8q + i/8, slot i%8 = logical chunk (i%8) ^ swz_b(row).
  // Columns past N are clamped onto the last 8 valid ones (never stored).
  {
    const pk_u32x4 rs = rsrc_words(B, (uint32_t)((size_t)K * N * 2));
    const int ninstr = K >> 3;  // 1 KiB each
    for (int q = wid; q < ninstr; q += RQ_THREADS / 64) {
      const int row = 8 * q + (lane >> 3), sl = lane & 7;
      const int col = min(n0 + 8 * (sl ^ swz_b<RQ_BN>(row)), N - 8);
      dma_lds16(rs, smem8 + q * 1024, (uint32_t)(((size_t)row * N + col) * 2), 0);
    }
  }

  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < RQ_XPT; ++j)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float a = lo_bf(xv[j][e]), b = hi_bf(xv[j][e]);
      ss += a * a;
      ss += b * b;
    }
#pragma unroll
  for (int o = 1; o < RQ_TPR; o <<= 1) ss += __shfl_xor(ss, o, 64);
  const float rms = sqrtf(ss * inv_cols + eps);
  // x / rms: the three-operation exact division (div_fast) when every
  // numerator and divisor of the wave is in its range, else the IEEE division
  DivSpan span;
  if (gm < M) {
#pragma unroll
    for (int j = 0; j < RQ_XPT; ++j)
      if (j < nxc)
#pragma unroll
        for (int e = 0; e < 4; ++e) div_span_add(span, xv[j][e]);
  }
  const bool fast = __all(div_row_ok(rms) && div_span_ok(span));
  auto normalise = [&](auto fast_c) __attribute__((always_inline)) {
    constexpr bool FAST = decltype(fast_c)::value;
    const float rinv = FAST ? 1.0f / rms : 0.f;
#pragma unroll
    for (int j = 0; j < RQ_XPT; ++j) {
      if (j < nxc) {
        const int c = c0 + RQ_TPR * j;
        u32x4 o;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          float a, b;
          if constexpr (FAST) {
            a = div_fast(lo_bf(xv[j][e]), rms, rinv);
            b = div_fast(hi_bf(xv[j][e]), rms, rinv);
          } else {
            a = lo_bf(xv[j][e]) / rms;
            b = hi_bf(xv[j][e]) / rms;
          }
          if (gamma) {
            a *= lo_bf(gv[j][e]);
            b *= hi_bf(gv[j][e]);
          }
          o[e] = pack_bf(a, b);
        }
        *reinterpret_cast<u32x4 *>(Ap + r * K + ((c ^ (r & 7)) << 3)) = o;
      }
    }
  };
  if (fast) normalise(std::true_type{});
  else normalise(std::false_type{});
  vm_wait<0>();     // this wave's W loads have landed
  __syncthreads();  // everyone's W loads and panel stores

  // ---- MFMA: wave -> (column block wid & 1, K part wid >> 1 of RQ_KP)
  const int cb = wid & 1, kp = wid >> 1;
  const int ks = K / (16 * RQ_KP);  // 16-k steps per part
  const int grp = lane >> 4, gi = lane & 15;
  const int b_krow = 8 * (grp >> 1) + (gi >> 2);
  const int b_col = cb * 32 + 16 * (grp & 1) + 4 * (gi & 3);
  const int a_row = lane & 31;
  f32x16 acc;
#pragma unroll
  for (int e = 0; e < 16; ++e) acc[e] = 0.f;
  for (int s = kp * ks; s < (kp + 1) * ks; ++s) {
    const int c = 2 * s + (lane >> 5);
    const bf16x8 af = lds_read_a(Ap + a_row * K + ((c ^ (a_row & 7)) << 3));
    i16x4 hb[2];
#pragma unroll
    for (int rr = 0; rr < 2; ++rr) {
      const int k = 16 * s + 4 * rr + b_krow;
      const int cc = b_col >> 3;
      hb[rr] = lds_read_tr(Bs + k * RQ_BN + ((cc ^ swz_b<RQ_BN>(k)) << 3) + (b_col & 7));
    }
    acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
        af, __builtin_bit_cast(bf16x8, __builtin_shufflevector(hb[0], hb[1], 0, 1, 2, 3, 4, 5, 6, 7)), acc, 0, 0,
        0);
  }
  // ---- add the K parts in order (part 0 + part 1 + ...) and store
  __syncthreads();  // everyone is done reading W: reuse its region (pk_panel_lds_bytes keeps >= 24 KiB)
  float *red = reinterpret_cast<float *>(Bs);  // [RQ_KP - 1][32][64] fp32
  if (kp > 0) {
#pragma unroll
    for (int i = 0; i < 16; ++i)
      red[(kp - 1) * RQ_BM * RQ_BN + ((i >> 2) * 8 + (lane >> 5) * 4 + (i & 3)) * RQ_BN + cb * 32 + (lane & 31)] = acc[i];
  }
  __syncthreads();
  if (kp == 0) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int o = ((i >> 2) * 8 + (lane >> 5) * 4 + (i & 3)) * RQ_BN + cb * 32 + (lane & 31);
      float v = acc[i];
#pragma unroll
      for (int q = 1; q < RQ_KP; ++q) v = v + red[(q - 1) * RQ_BM * RQ_BN + o];
      red[o] = v;
    }
  }
  __syncthreads();
  if (tid < RQ_BM * 8) {
    const int rr = tid >> 3, c8 = (tid & 7) * 8;
    const int m = m0 + rr, n = n0 + c8;
    if (m < M && n < N) {
      const float *p = red + rr * RQ_BN + c8;
      const u32x4 o = {pack_bf(p[0], p[1]), pack_bf(p[2], p[3]), pack_bf(p[4], p[5]), pack_bf(p[6], p[7])};
      *reinterpret_cast<u32x4 *>(C + (size_t)m * N + n) = o;
    }
  }
}

}  // namespace gk
}  // namespace pk
