// attention_kernels.hpp -- the attention kernels for gfx950 (bodies), shared
// by the library (attention.hip, which wraps them as __global__ kernels) and
// by code objects the emitter instantiates at a tuned configuration
// (csrc/runtime/codegen.cpp).  Both compile this one source.
//
// Arithmetic of kernels/cpu/attention.cpp:95-163: for query i of a (b,h) the
// visible keys are j <= S_kv - S_q + i (causal) or all j; score = (q.k) * scale
// in fp32; softmax in fp32; o = bf16(sum_j p_j v_j / sum_j p_j).
#pragma once

#include "attention_args.h"
#include "pk_common.hpp"

namespace pk {
namespace att {

// Kernel arguments: the C structs of attention_args.h (host and device share them).
using AttArgs = pk_att_args;
using FaArgs = pk_fa_args;

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) i16x4 lds_i16x4;

constexpr int AT_WAVES = 4;
constexpr int AT_BQ = AT_WAVES * 32;
constexpr int AT_BKV = 64;
constexpr int AT_THREADS = AT_WAVES * 64;


// V rows: 16-byte-chunk XOR so the 4 rows of one 16-lane transpose read hit
// distinct banks (rows of 64 B pair up in one 128-byte bank sweep when DP = 32).
template <int DP>
__device__ __forceinline__ int swz_v(int k) {
  if constexpr (DP >= 128) {
    // 0, 4, 10, 14 for k & 3 = 0..3, as arithmetic: a table would live in
    // memory and be re-read (with a wait on every load in flight) after
    // each barrier of the pipelined loops
    const int j = k & 3;
    return (j << 2) | ((j >> 1) << 1);
  } else if constexpr (DP == 64) {
    return (k & 3) * 2;
  } else {
    return ((k >> 1) & 1) * 2;
  }
}

// K rows: XOR the chunk index with row bits so the 16 consecutive rows one
// ds_read_b128 group reads (16 lanes = 256 B of the 64 x 4-byte banks) hit
// distinct banks: 256-byte rows (16 chunks) take row & 15; 128-byte rows
// (8 chunks) split by row parity into bank halves and take (row >> 1) & 7;
// 64-byte rows take (row >> 2) & 3.
template <int CH>
__device__ __forceinline__ int swz_k(int c, int row) {
  if constexpr (CH >= 16) return (c & ~15) | ((c & 15) ^ (row & 15));
  else if constexpr (CH == 8) return c ^ ((row >> 1) & 7);
  else return c ^ ((row >> 2) & 3);
}

template <int DP, bool ALIGNED>
__device__ __forceinline__ void att_body(AttArgs g) {
  constexpr int CH = DP / 8;                 // 16-byte chunks per row
  constexpr int TILE_CHUNKS = AT_BKV * CH;   // per K or V tile
  constexpr int LC = TILE_CHUNKS / AT_THREADS;
  constexpr int DS = DP / 16;                // k-steps of the QK^T product
  constexpr int DB = DP / 32;                // d blocks of the PV product
  static_assert(TILE_CHUNKS % AT_THREADS == 0, "tile/thread mismatch");

  __shared__ __attribute__((aligned(16))) uint16_t Ks[2][AT_BKV * DP];
  __shared__ __attribute__((aligned(16))) uint16_t Vs[2][AT_BKV * DP];

  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  // Block -> (bh, q tile, split): consecutive blocks share (bh) so the 8 XCDs
  // each get whole heads when the grid divides evenly.
  int b = blockIdx.x;
  const int per_bh = g.q_tiles * g.splits;
  const int total = g.BH * per_bh;
  if ((total & 7) == 0) b = (b & 7) * (total >> 3) + (b >> 3);
  const int bh = b / per_bh;
  const int rem = b % per_bh;
  const int qt = rem / g.splits, split = rem % g.splits;
  const int q0 = qt * AT_BQ;
  const int qw = q0 + wid * 32;
  const int my_q = qw + (lane & 31);

  // visible key range of this query tile, then this split's share
  const int off = g.S_kv - g.S_q;
  int kv_end = g.S_kv;
  if (g.causal) kv_end = min(g.S_kv, max(0, off + q0 + AT_BQ));
  const int ntiles = (kv_end + AT_BKV - 1) / AT_BKV;
  const int tps = (ntiles + g.splits - 1) / g.splits;
  const int t_begin = split * tps;
  const int t_end = min(ntiles, t_begin + tps);

  const size_t kvbase = (size_t)bh * g.kv_rows * g.D;
  const uint16_t *Kp = g.K + kvbase;
  const uint16_t *Vp = g.V + kvbase;

  // Q^T fragments (B operand): lane -> query lane%32, d = 16*ds + 8*(lane/32) + 0..7.
  bf16x8 qf[DS];
  {
    const uint16_t *qrow = g.Q + ((size_t)bh * g.S_q + my_q) * g.D;
#pragma unroll
    for (int ds = 0; ds < DS; ++ds) {
      const int d = 16 * ds + 8 * (lane >> 5);
      u32x4 v = {0, 0, 0, 0};
      if (my_q < g.S_q) {
        if constexpr (ALIGNED) {
          if (d < g.D) v = *reinterpret_cast<const u32x4 *>(qrow + d);
        } else {
#pragma unroll
          for (int e = 0; e < 8; ++e)
            if (d + e < g.D) v[e >> 1] |= (uint32_t)qrow[d + e] << (16 * (e & 1));
        }
      }
      qf[ds] = __builtin_bit_cast(bf16x8, v);
    }
  }

  u32x4 rk[LC], rv[LC];
  auto load_kv = [&](int t) {
    const int k0 = t * AT_BKV;
#pragma unroll
    for (int i = 0; i < LC; ++i) {
      const int q = tid + i * AT_THREADS, row = q / CH, c = q % CH;
      const int key = k0 + row, d = c * 8;
      u32x4 a = {0, 0, 0, 0}, v = {0, 0, 0, 0};
      if (key < kv_end) {
        const size_t o = (size_t)key * g.D + d;
        if constexpr (ALIGNED) {
          if (d < g.D) {
            a = *reinterpret_cast<const u32x4 *>(Kp + o);
            v = *reinterpret_cast<const u32x4 *>(Vp + o);
          }
        } else {
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            if (d + e < g.D) {
              a[e >> 1] |= (uint32_t)Kp[o + e] << (16 * (e & 1));
              v[e >> 1] |= (uint32_t)Vp[o + e] << (16 * (e & 1));
            }
          }
        }
      }
      rk[i] = a;
      rv[i] = v;
    }
  };
  auto store_kv = [&](int s) {
#pragma unroll
    for (int i = 0; i < LC; ++i) {
      const int q = tid + i * AT_THREADS, row = q / CH, c = q % CH;
      *reinterpret_cast<u32x4 *>(&Ks[s][row * DP + (swz_k<CH>(c, row) << 3)]) = rk[i];
      *reinterpret_cast<u32x4 *>(&Vs[s][row * DP + ((c ^ swz_v<DP>(row)) << 3)]) = rv[i];
    }
  };

  f32x16 acc_o[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db)
#pragma unroll
    for (int e = 0; e < 16; ++e) acc_o[db][e] = 0.f;
  float m_run = -INFINITY, l_run = 0.f;
  const int q_limit = g.causal ? (off + my_q) : (g.S_kv - 1);

  const int grp = lane >> 4, gi = lane & 15, h = lane >> 5;

  if (t_begin < t_end) {
    load_kv(t_begin);
    store_kv(0);
  }
  __syncthreads();
  // The next tile is staged through registers.  Up to D = 128 its loads stay
  // in flight during this tile's products (stored to LDS at the end); at
  // D = 256 the accumulators and Q fragments fill the register file, so the
  // next tile is loaded and stored at once, into the buffer no one reads in
  // this iteration.
  constexpr bool kOverlapLoads = DP <= 128;
  for (int t = t_begin; t < t_end; ++t) {
    const int cur = (t - t_begin) & 1;
    if (t + 1 < t_end) {
      load_kv(t + 1);
      if constexpr (!kOverlapLoads) store_kv(cur ^ 1);
    }
    const uint16_t *ks = Ks[cur];
    const uint16_t *vs = Vs[cur];
    const int k0 = t * AT_BKV;

    // ---- S^T = K Q^T for 64 keys (2 blocks of 32)
    f32x16 s[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
      for (int e = 0; e < 16; ++e) s[kb][e] = 0.f;
      const int row = kb * 32 + (lane & 31);
#pragma unroll
      for (int ds = 0; ds < DS; ++ds) {
        const int c = 2 * ds + h;
        const u32x4 kv = *reinterpret_cast<const u32x4 *>(ks + row * DP + (swz_k<CH>(c, row) << 3));
        s[kb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, kv), qf[ds],
                                                        s[kb], 0, 0, 0);
      }
    }
    // ---- scale, mask, online softmax (this lane: one query, 32 keys)
    float tmax = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int key = k0 + kb * 32 + (i >> 2) * 8 + h * 4 + (i & 3);
        float v = s[kb][i] * g.scale;
        if (key > q_limit || key >= kv_end) v = -INFINITY;
        s[kb][i] = v;
        tmax = fmaxf(tmax, v);
      }
    tmax = xor32_max(tmax);
    const float m_new = fmaxf(m_run, tmax);
    const float m_use = (m_new == -INFINITY) ? 0.f : m_new;
    const float alpha = __expf(m_run - m_use);
    // p in fp32 (the sum uses it unrounded, as the reference does); for the PV
    // product p = p_hi + p_lo with both halves bf16, so the MFMA sees p to
    // ~2^-17 relative instead of the 2^-9 of a single bf16.
    float psum = 0.f;
    uint32_t phi[2][8], plo[2][8];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int i = 0; i < 16; i += 2) {
        const float p0 = __expf(s[kb][i] - m_use);
        const float p1 = __expf(s[kb][i + 1] - m_use);
        psum += p0 + p1;
        const uint32_t h0 = f2bf(p0), h1 = f2bf(p1);
        const uint32_t l0 = f2bf(p0 - bf2f(h0)), l1 = f2bf(p1 - bf2f(h1));
        phi[kb][i >> 1] = h0 | (h1 << 16);
        plo[kb][i >> 1] = l0 | (l1 << 16);
      }
    psum = xor32_sum(psum);
    l_run = l_run * alpha + psum;
    m_run = m_new;
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc_o[db][e] *= alpha;

    // ---- O^T += V^T (P_hi + P_lo)^T over 4 steps of 16 keys
#pragma unroll
    for (int st = 0; st < 4; ++st) {
      const int kb = st >> 1, hf = st & 1;
      const u32x4 hv4 = {phi[kb][4 * hf + 0], phi[kb][4 * hf + 1], phi[kb][4 * hf + 2], phi[kb][4 * hf + 3]};
      const u32x4 lv4 = {plo[kb][4 * hf + 0], plo[kb][4 * hf + 1], plo[kb][4 * hf + 2], plo[kb][4 * hf + 3]};
      const bf16x8 pb_hi = __builtin_bit_cast(bf16x8, hv4);
      const bf16x8 pb_lo = __builtin_bit_cast(bf16x8, lv4);
#pragma unroll
      for (int db = 0; db < DB; ++db) {
        i16x4 hv[2];
#pragma unroll
        for (int r = 0; r < 2; ++r) {
          const int key = st * 16 + 8 * r + 4 * h + (gi >> 2);
          const int d = db * 32 + 16 * (grp & 1) + 4 * (gi & 3);
          const int c = d >> 3;
          hv[r] = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (lds_i16x4 *)(vs + key * DP + ((c ^ swz_v<DP>(key)) << 3) + (d & 7)));
        }
        short tmp[8] = {hv[0][0], hv[0][1], hv[0][2], hv[0][3], hv[1][0], hv[1][1], hv[1][2], hv[1][3]};
        const bf16x8 va = __builtin_bit_cast(bf16x8, tmp);
        acc_o[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(va, pb_hi, acc_o[db], 0, 0, 0);
        acc_o[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(va, pb_lo, acc_o[db], 0, 0, 0);
      }
    }
    if constexpr (kOverlapLoads)
      if (t + 1 < t_end) store_kv(cur ^ 1);
    __syncthreads();
  }

  // ---- output: acc_o[db][i] -> d = db*32 + (i/4)*8 + h*4 + i%4, query my_q
  if (my_q >= g.S_q) return;
  const size_t orow = (size_t)bh * g.S_q + my_q;
  if (g.splits == 1) {
    const float inv = 1.0f / l_run;
    uint16_t *op = g.O + orow * g.D;
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int d = db * 32 + (i >> 2) * 8 + h * 4 + (i & 3);
        if (d < g.D) op[d] = (uint16_t)f2bf(acc_o[db][i] * inv);
      }
  } else {
    float *po = g.part_o + ((size_t)split * g.BH * g.S_q + orow) * DP;
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int i = 0; i < 16; ++i) po[db * 32 + (i >> 2) * 8 + h * 4 + (i & 3)] = acc_o[db][i];
    if (h == 0) {
      float *pml = g.part_ml + ((size_t)split * g.BH * g.S_q + orow) * 2;
      pml[0] = m_run;
      pml[1] = l_run;
    }
  }
}

// ---------------------------------------------------------------------------
// Wide heads (256 < D <= 1024, attention_prefill.cu:166-180 accepts any D up
// to 1024).  A workgroup of 4 waves owns 32 queries of one (b,h); wave w owns
// head dims [256 w, 256 w + 256).  Per step of 32 keys: the K and V rows go to
// LDS (zero past D), each wave forms the partial scores of its dims
// (S^T = K Q^T, 16 MFMA k-steps) into LDS, then every wave adds the partials
// in wave order, runs the online softmax of att_body on the full scores (the
// same values in every wave) and accumulates P V for its own dims.  Waves
// whose dims lie past D skip the products.  Key splits and their merge as in
// att_body (att_combine_body<AW_DMAX>).
constexpr int AW_BQ = 32, AW_BKV = 32, AW_DMAX = 1024, AW_DC = 256, AW_WAVES = 4;
constexpr int AW_THREADS = AW_WAVES * 64;

template <bool ALIGNED>
__device__ __forceinline__ void att_wide_body(AttArgs g) {
  constexpr int DS = AW_DC / 16;   // k-steps of a wave's partial scores
  constexpr int DB = AW_DC / 32;   // d blocks of a wave's P V product
  constexpr int KS = AW_DMAX + 8;  // LDS row strides (elements): consecutive K rows
  constexpr int VS = AW_DMAX + 16; // 16 B apart in the banks, V rows 32 B
  __shared__ __attribute__((aligned(16))) uint16_t Ks[AW_BKV * KS];
  __shared__ __attribute__((aligned(16))) uint16_t Vs[AW_BKV * VS];
  __shared__ float Sp[AW_WAVES][16][64];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int h = lane >> 5, grp = lane >> 4, gi = lane & 15;
  int b = blockIdx.x;
  const int per_bh = g.q_tiles * g.splits;
  const int total = g.BH * per_bh;
  if ((total & 7) == 0) b = (b & 7) * (total >> 3) + (b >> 3);
  const int bh = b / per_bh;
  const int rem = b % per_bh;
  const int qt = rem / g.splits, split = rem % g.splits;
  const int q0 = qt * AW_BQ;
  const int my_q = q0 + (lane & 31);

  const int off = g.S_kv - g.S_q;
  int kv_end = g.S_kv;
  if (g.causal) kv_end = min(g.S_kv, max(0, off + q0 + AW_BQ));
  const int ntiles = (kv_end + AW_BKV - 1) / AW_BKV;
  const int tps = (ntiles + g.splits - 1) / g.splits;
  const int t_begin = split * tps;
  const int t_end = min(ntiles, t_begin + tps);

  const int nc = (g.D + AW_DC - 1) / AW_DC;  // waves that own dims
  const int dw = wid * AW_DC;                // this wave's first dim
  const bool active = wid < nc;
  const int cpr = nc * AW_DC / 8;            // 16-byte chunks of an LDS row in use

  const size_t kvbase = (size_t)bh * g.kv_rows * g.D;
  const uint16_t *Kp = g.K + kvbase;
  const uint16_t *Vp = g.V + kvbase;

  // Q^T fragments of this wave's dims: query lane % 32, d = dw + 16 ds + 8 h + 0..7
  bf16x8 qf[DS];
  {
    const uint16_t *qrow = g.Q + ((size_t)bh * g.S_q + min(my_q, g.S_q - 1)) * g.D;
#pragma unroll
    for (int ds = 0; ds < DS; ++ds) {
      const int d = dw + 16 * ds + 8 * h;
      u32x4 v = {0, 0, 0, 0};
      if (my_q < g.S_q) {
        if constexpr (ALIGNED) {
          if (d < g.D) v = *reinterpret_cast<const u32x4 *>(qrow + d);
        } else {
#pragma unroll
          for (int e = 0; e < 8; ++e)
            if (d + e < g.D) v[e >> 1] |= (uint32_t)qrow[d + e] << (16 * (e & 1));
        }
      }
      qf[ds] = __builtin_bit_cast(bf16x8, v);
    }
  }

  // K and V rows [k0, k0 + 32) into LDS, zero past kv_end and past D
  auto load_tile = [&](int t) {
    const int k0 = t * AW_BKV;
    for (int q = tid; q < AW_BKV * cpr; q += AW_THREADS) {
      const int row = q / cpr, d = 8 * (q % cpr), key = k0 + row;
      u32x4 a = {0, 0, 0, 0}, v = {0, 0, 0, 0};
      if (key < kv_end && d < g.D) {
        const size_t o = (size_t)key * g.D + d;
        if constexpr (ALIGNED) {
          a = *reinterpret_cast<const u32x4 *>(Kp + o);
          v = *reinterpret_cast<const u32x4 *>(Vp + o);
        } else {
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            if (d + e < g.D) {
              a[e >> 1] |= (uint32_t)Kp[o + e] << (16 * (e & 1));
              v[e >> 1] |= (uint32_t)Vp[o + e] << (16 * (e & 1));
            }
          }
        }
      }
      *reinterpret_cast<u32x4 *>(&Ks[row * KS + d]) = a;
      *reinterpret_cast<u32x4 *>(&Vs[row * VS + d]) = v;
    }
  };

  f32x16 acc_o[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db)
#pragma unroll
    for (int e = 0; e < 16; ++e) acc_o[db][e] = 0.f;
  float m_run = -INFINITY, l_run = 0.f;
  const int q_limit = g.causal ? (off + my_q) : (g.S_kv - 1);

  for (int t = t_begin; t < t_end; ++t) {
    __syncthreads();  // the previous step's reads of Ks, Vs and Sp are done
    load_tile(t);
    __syncthreads();
    const int k0 = t * AW_BKV;
    if (active) {
      // partial S^T over this wave's dims (32 keys x 32 queries)
      f32x16 sp;
#pragma unroll
      for (int e = 0; e < 16; ++e) sp[e] = 0.f;
      const int row = lane & 31;
#pragma unroll
      for (int ds = 0; ds < DS; ++ds) {
        const u32x4 kv = *reinterpret_cast<const u32x4 *>(&Ks[row * KS + dw + 16 * ds + 8 * h]);
        sp = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, kv), qf[ds], sp, 0, 0, 0);
      }
#pragma unroll
      for (int e = 0; e < 16; ++e) Sp[wid][e][lane] = sp[e];
    }
    __syncthreads();
    if (!active) continue;  // wave-uniform; every wave still meets the barriers above

    // ---- full scores (partials added in wave order), scale, mask, online softmax
    float tmax = -INFINITY;
    float s[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      float v = Sp[0][i][lane];
      for (int w = 1; w < nc; ++w) v += Sp[w][i][lane];
      const int key = k0 + (i >> 2) * 8 + h * 4 + (i & 3);
      v *= g.scale;
      if (key > q_limit || key >= kv_end) v = -INFINITY;
      s[i] = v;
      tmax = fmaxf(tmax, v);
    }
    tmax = xor32_max(tmax);
    const float m_new = fmaxf(m_run, tmax);
    const float m_use = (m_new == -INFINITY) ? 0.f : m_new;
    const float alpha = __expf(m_run - m_use);
    // p = p_hi + p_lo with both halves bf16 for the P V product (as att_body)
    float psum = 0.f;
    uint32_t phi[8], plo[8];
#pragma unroll
    for (int i = 0; i < 16; i += 2) {
      const float p0 = __expf(s[i] - m_use);
      const float p1 = __expf(s[i + 1] - m_use);
      psum += p0 + p1;
      const uint32_t h0 = f2bf(p0), h1 = f2bf(p1);
      const uint32_t l0 = f2bf(p0 - bf2f(h0)), l1 = f2bf(p1 - bf2f(h1));
      phi[i >> 1] = h0 | (h1 << 16);
      plo[i >> 1] = l0 | (l1 << 16);
    }
    psum = xor32_sum(psum);
    l_run = l_run * alpha + psum;
    m_run = m_new;
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc_o[db][e] *= alpha;

    // ---- O^T += V^T (P_hi + P_lo)^T for this wave's dims, 2 steps of 16 keys
#pragma unroll
    for (int st = 0; st < 2; ++st) {
      const u32x4 hv4 = {phi[4 * st + 0], phi[4 * st + 1], phi[4 * st + 2], phi[4 * st + 3]};
      const u32x4 lv4 = {plo[4 * st + 0], plo[4 * st + 1], plo[4 * st + 2], plo[4 * st + 3]};
      const bf16x8 pb_hi = __builtin_bit_cast(bf16x8, hv4);
      const bf16x8 pb_lo = __builtin_bit_cast(bf16x8, lv4);
#pragma unroll
      for (int db = 0; db < DB; ++db) {
        i16x4 hv[2];
#pragma unroll
        for (int r = 0; r < 2; ++r) {
          const int key = st * 16 + 8 * r + 4 * h + (gi >> 2);
          const int d = dw + db * 32 + 16 * (grp & 1) + 4 * (gi & 3);
          hv[r] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4 *)(&Vs[key * VS + d]));
        }
        const bf16x8 va = __builtin_bit_cast(bf16x8, __builtin_shufflevector(hv[0], hv[1], 0, 1, 2, 3, 4, 5, 6, 7));
        acc_o[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(va, pb_hi, acc_o[db], 0, 0, 0);
        acc_o[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(va, pb_lo, acc_o[db], 0, 0, 0);
      }
    }
  }

  // ---- output: acc_o[db][i] -> d = dw + db*32 + (i/4)*8 + h*4 + i%4, query my_q
  if (!active || my_q >= g.S_q) return;
  const size_t orow = (size_t)bh * g.S_q + my_q;
  if (g.splits == 1) {
    const float inv = 1.0f / l_run;
    uint16_t *op = g.O + orow * g.D;
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int d = dw + db * 32 + (i >> 2) * 8 + h * 4 + (i & 3);
        if (d < g.D) op[d] = (uint16_t)f2bf(acc_o[db][i] * inv);
      }
  } else {
    float *po = g.part_o + ((size_t)split * g.BH * g.S_q + orow) * AW_DMAX;
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int d = dw + db * 32 + (i >> 2) * 8 + h * 4 + (i & 3);
        if (d < g.D) po[d] = acc_o[db][i];
      }
    if (wid == 0 && h == 0) {
      float *pml = g.part_ml + ((size_t)split * g.BH * g.S_q + orow) * 2;
      pml[0] = m_run;
      pml[1] = l_run;
    }
  }
}

template <int DP>
__device__ __forceinline__ void att_combine_body(AttArgs g) {
  const int64_t rows = (int64_t)g.BH * g.S_q;
  const int64_t total = rows * g.D;
  for (int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x; t < total; t += (int64_t)gridDim.x * 256) {
    const int64_t row = t / g.D;
    const int d = (int)(t % g.D);
    float M = -INFINITY;
    for (int s = 0; s < g.splits; ++s) M = fmaxf(M, g.part_ml[((size_t)s * rows + row) * 2]);
    const float Mu = (M == -INFINITY) ? 0.f : M;
    float L = 0.f, acc = 0.f;
    for (int s = 0; s < g.splits; ++s) {
      const float m = g.part_ml[((size_t)s * rows + row) * 2];
      const float l = g.part_ml[((size_t)s * rows + row) * 2 + 1];
      const float w = __expf(m - Mu);
      L += l * w;
      acc += g.part_o[((size_t)s * rows + row) * DP + d] * w;
    }
    g.O[row * g.D + d] = (uint16_t)f2bf(acc * (1.0f / L));
  }
}

// ---------------------------------------------------------------------------
// Flash-style prefill for head dims 64 and 128 (the config-3 path).
//
// A workgroup of 8 waves owns 32*QG queries of one (b,h) and walks its key
// range in steps of 32*KH keys (QG * KH = 8): wave (qg, kh) handles query
// group qg (32 queries, the S^T layout above) against keys
// [step*32*KH + 32*kh, +32) with its own running max / sum / accumulator.
// Tile shapes: QG 4 (128 queries x 64 keys per step) or QG 2 (64 x 128).
// Two waves share each SIMD.  K and V tiles arrive by buffer_load ... lds
// (waves 0-3 load K, 4-7 V) into two rings of 64 KiB, one barrier per step;
// within a wave the score MFMAs of the next step and the P V MFMAs of the
// previous one overlap the softmax of the current step.  Diagonal blocks
// are masked, blocks above the diagonal skipped.  At the end the KH partial
// states of each query are merged in LDS in kh order.  When the grid would
// not fill the chip, the key range is also split over `splits` workgroups
// whose fp32 partials fa_combine_kernel merges in split order.
// Fused KV append: rows >= S_cache are read from K_new/V_new directly and the
// kernel also copies them into the cache (no reader of the cache needs them,
// so the copy is unordered).
constexpr int FA_WAVES = 8;
constexpr int FA_THREADS = FA_WAVES * 64;
constexpr int FA_RING = 128 * 1024;  // bytes of LDS ring


template <int DP, int QG, bool FUSED>
__device__ __forceinline__ void fa_body(FaArgs g) {
  constexpr int KH = FA_WAVES / QG;          // key blocks of 32 per step
  constexpr int BQ = 32 * QG;                // queries per workgroup
  constexpr int BKV = 32 * KH;               // keys per step
  constexpr int CH = DP / 8;                 // 16-byte chunks per row
  constexpr int TB = BKV * DP * 2;           // bytes of one K (or V) tile
  constexpr int SL = FA_RING / (2 * TB);     // slots of the K ring and of the V ring
  constexpr int NK = TB / 1024;              // DMA instructions per tile
  constexpr int NPW = NK / (FA_WAVES / 2);   // per wave per step
  constexpr int RPI = 1024 / (2 * DP);       // rows per DMA instruction
  constexpr int DS = DP / 16, DB = DP / 32;
  static_assert(SL >= 2 && NPW >= 1 && NK % (FA_WAVES / 2) == 0, "ring shape");
  constexpr int PS = DP + 4;                 // merge-buffer row stride (floats), 16 B padding
  constexpr int MERGE = FA_WAVES * 32 * PS * 4;
  // the ring, reused as the merge buffer after the last step
  __shared__ __attribute__((aligned(1024))) uint8_t ring[MERGE > FA_RING ? MERGE : FA_RING];
  __shared__ float ml_s[FA_WAVES][32][2];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int qg = wid % QG, kh = wid / QG;
  // arguments used in the loop, read once
  const float scale = g.scale;
  const bool causal = g.causal != 0;
  const int S_cache = g.S_cache;
  const int h = lane >> 5, grp = lane >> 4, gi = lane & 15;
  int b = blockIdx.x;
  const int per_bh = g.q_tiles * g.splits;
  const int total = g.BH * per_bh;
  if ((total & 7) == 0) b = (b & 7) * (total >> 3) + (b >> 3);
  const int bh = b / per_bh, rem = b % per_bh;
  const int qt = rem / g.splits, split = rem % g.splits;
  const int q0 = qt * BQ;
  const int qw = q0 + 32 * qg;
  const int my_q = qw + (lane & 31);
  const int off = g.S_kv - g.S_q;
  const int kv_end = causal ? min(g.S_kv, max(0, off + q0 + BQ)) : g.S_kv;
  const int ntiles = (kv_end + BKV - 1) / BKV;
  const int tps = (ntiles + g.splits - 1) / g.splits;
  const int t_begin = min(ntiles, split * tps);
  const int nsteps = min(ntiles, t_begin + tps) - t_begin;
  const int S_new = g.S_kv - S_cache;

  // ---- fused append: this workgroup's share of the new rows -> cache
  if (FUSED) {
    const int64_t per_head = (int64_t)S_new * DP / 8;  // 16-byte units
    const int64_t units = (int64_t)g.BH * per_head;
    for (int64_t u = (int64_t)blockIdx.x * FA_THREADS + tid; u < units; u += (int64_t)gridDim.x * FA_THREADS) {
      const int64_t hd = u / per_head, r = u % per_head;
      const size_t src = (size_t)hd * S_new * DP + (size_t)r * 8;
      const size_t dst = ((size_t)hd * g.kv_rows + S_cache) * DP + (size_t)r * 8;
      *reinterpret_cast<u32x4 *>(g.Kc + dst) = *reinterpret_cast<const u32x4 *>(g.Kn + src);
      *reinterpret_cast<u32x4 *>(g.Vc + dst) = *reinterpret_cast<const u32x4 *>(g.Vn + src);
    }
  }

  // ---- Q^T fragments (B operand): query lane % 32, d = 16 ds + 8 h + 0..7
  bf16x8 qf[DS];
  {
    const uint16_t *qrow = g.Q + ((size_t)bh * g.S_q + min(my_q, g.S_q - 1)) * DP;
#pragma unroll
    for (int ds = 0; ds < DS; ++ds) {
      u32x4 v = *reinterpret_cast<const u32x4 *>(qrow + 16 * ds + 8 * h);
      if (my_q >= g.S_q) v = u32x4{0, 0, 0, 0};
      qf[ds] = __builtin_bit_cast(bf16x8, v);
    }
  }

  // ---- DMA: per head, the cache rows and (FUSED) the new rows; with FUSED,
  // S_cache is a multiple of BKV, so a step reads one source.  Waves 0-3 load
  // the K tile, waves 4-7 the V tile, NPW 1 KiB instructions each;
  // instruction qq covers tile rows qq*RPI .. qq*RPI+RPI-1.  The per-lane
  // offset inside the tile is loop-invariant and the step's first row goes
  // into the scalar offset; only a step that reaches past kv_end clamps rows
  // (onto the last visible row: finite data, masked).
  const bool isk = wid < FA_WAVES / 2;
  const int wq = isk ? wid : wid - FA_WAVES / 2;
  const uint16_t *src_c = (isk ? g.K : g.V) + (size_t)bh * g.kv_rows * DP;
  const uint16_t *src_n = FUSED ? (isk ? g.Kn : g.Vn) + (size_t)bh * S_new * DP : src_c;
  const pk_u32x4 rs_c = rsrc_words(src_c, (uint32_t)((size_t)g.kv_rows * DP * 2));
  const pk_u32x4 rs_n = rsrc_words(src_n, FUSED ? (uint32_t)((size_t)S_new * DP * 2) : 0u);
  // Lane offset of instruction j: row (wq*NPW + j)*RPI + lane/CH, swizzled
  // chunk lc.  RPI rows are 1 KiB and the swizzles see at most row & 15 (K)
  // or row & 3 (V), so the offset is vb[j % VP] + 1024*j (the 1024*j goes
  // into the scalar offset): VP registers instead of NPW.
  constexpr int VP = RPI >= 16 ? 1 : 16 / RPI > 4 ? 4 : 16 / RPI;
  static_assert(RPI * DP * 2 == 1024 && NPW % VP == 0, "DMA row blocks");
  uint32_t vb[VP];
#pragma unroll
  for (int p = 0; p < VP; ++p) {
    const int row = (wq * NPW + p) * RPI + lane / CH, sl = lane % CH;
    const int lc = isk ? swz_k<CH>(sl, row) : (sl ^ swz_v<DP>(row));
    vb[p] = (uint32_t)(row * DP * 2 + 16 * lc - 1024 * p);
  }
  auto issue = [&](int step, int slot) __attribute__((always_inline)) {
    const int k0 = (t_begin + step) * BKV;
    const bool nw = FUSED && k0 >= S_cache;
    const pk_u32x4 rs = nw ? rs_n : rs_c;
    const int r0 = nw ? k0 - S_cache : k0;  // first row of the step in its source
    uint8_t *tile = ring + (isk ? slot : SL + slot) * TB;
    if (k0 + BKV <= kv_end) {
#pragma unroll
      for (int j = 0; j < NPW; ++j)
        dma_lds16(rs, tile + (wq * NPW + j) * 1024, vb[j % VP], (uint32_t)(r0 * DP * 2 + 1024 * j));
    } else {
#pragma unroll
      for (int j = 0; j < NPW; ++j) {
        const int row = (wq * NPW + j) * RPI + lane / CH;
        const int over = max(0, k0 + row - (kv_end - 1));  // rows past the last visible one
        dma_lds16(rs, tile + (wq * NPW + j) * 1024, vb[j % VP] - (uint32_t)(over * DP * 2),
                  (uint32_t)(r0 * DP * 2 + 1024 * j));
      }
    }
  };
  // instructions [j0, j1) of the DMA of a step that lies wholly below kv_end
  auto issue_rows = [&](int step, int slot, int j0, int j1) __attribute__((always_inline)) {
    const int k0 = (t_begin + step) * BKV;
    const bool nw = FUSED && k0 >= S_cache;
    const pk_u32x4 rs = nw ? rs_n : rs_c;
    const int r0 = nw ? k0 - S_cache : k0;
    uint8_t *tile = ring + (isk ? slot : SL + slot) * TB;
#pragma unroll
    for (int j = j0; j < j1; ++j)
      dma_lds16(rs, tile + (wq * NPW + j) * 1024, vb[j % VP], (uint32_t)(r0 * DP * 2 + 1024 * j));
  };

  f32x16 acc_o[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db)
#pragma unroll
    for (int e = 0; e < 16; ++e) acc_o[db][e] = 0.f;
  float m_run = -INFINITY, l_run = 0.f;
  const int q_limit = causal ? (off + my_q) : (g.S_kv - 1);
  const float c2 = scale * 1.4426950408889634f;  // scale * log2(e)

  // ---- one wave's block of a step: keys [kb0, kb0+32) x its 32 queries
  auto kb0_of = [&](int step) __attribute__((always_inline)) { return (t_begin + step) * BKV + 32 * kh; };
  // keys of the block visible to at least one of the wave's queries?
  auto visible = [&](int step) __attribute__((always_inline)) {
    const int kb0 = kb0_of(step);
    return kb0 < kv_end && !(causal && kb0 > off + qw + 31);
  };
  // does any key of the block need masking for some query of the wave?
  auto masked = [&](int step) __attribute__((always_inline)) {
    const int kb0 = kb0_of(step);
    return kb0 + 31 >= kv_end || (causal && kb0 + 31 > off + qw);
  };
  // S^T block = K Q^T (raw scores, unscaled)
  auto qk = [&](int slot) __attribute__((always_inline)) -> f32x16 {
    const uint8_t *ks = ring + slot * TB;
    f32x16 sc{};
    const int row = 32 * kh + (lane & 31);
#pragma unroll
    for (int ds = 0; ds < DS; ++ds) {
      const u32x4 kv = *reinterpret_cast<const u32x4 *>(ks + row * DP * 2 + 16 * swz_k<CH>(2 * ds + h, row));
      sc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, kv), qf[ds], sc, 0, 0, 0);
    }
    return sc;
  };
  // Softmax in the log2 domain on unscaled scores: p = 2^(s c - m c) with
  // c = scale * log2(e) (one FMA and v_exp_f32 per score).  The running max m
  // used in the exponent is raised only when a new score exceeds it by more
  // than 8 / c (p may reach 2^8 meanwhile); o = sum p v / sum p does not
  // depend on it, and skipping most rescales saves the multiply of the whole
  // accumulator.  Each weight is split into bf16 halves p = p_hi + p_lo for
  // the P V product.  MASKED is a compile-time flag so blocks off the
  // diagonal carry no mask arithmetic.  Returns the factor the accumulator
  // must be multiplied by (after the products of earlier steps are in it),
  // 1 when the max did not move.
  struct Pw {
    bf16x8 hi[2], lo[2];
  };
  auto row_max = [&](const f32x16 &x) __attribute__((always_inline)) {
    float m = -INFINITY;
#pragma unroll
    for (int i = 0; i < 16; ++i) m = fmaxf(m, x[i]);
    return xor32_max(m);
  };
  // pre_max: the block's row max when the caller has it (unmasked blocks)
  auto softmax = [&](auto mask_c, int step, f32x16 sc, Pw &pw, bool &resc, const float *pre_max = nullptr)
      __attribute__((always_inline)) -> float {
    constexpr bool MASKED = decltype(mask_c)::value;
    float tmax = -INFINITY;
    if (!MASKED && pre_max) {
      tmax = *pre_max;
    } else {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        if constexpr (MASKED) {
          const int key = kb0_of(step) + (i >> 2) * 8 + h * 4 + (i & 3);
          if (key > q_limit || key >= kv_end) sc[i] = -INFINITY;
        }
        tmax = fmaxf(tmax, sc[i]);
      }
      tmax = xor32_max(tmax);
    }
    float alpha = 1.f;
    resc = __any((tmax - m_run) * c2 > 8.0f);  // also true for the first block (m_run = -inf)
    if (resc) {
      const float m_new = fmaxf(m_run, tmax);
      alpha = m_run == -INFINITY ? 0.f : __builtin_amdgcn_exp2f((m_run - m_new) * c2);
      m_run = m_new;
    }
    const float mc = m_run == -INFINITY ? 0.f : m_run * c2;
    float psum = 0.f;
    uint32_t phi[8], plo[8];
#pragma unroll
    for (int i = 0; i < 16; i += 2) {
      const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[i], c2, -mc));
      const float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[i + 1], c2, -mc));
      psum += p0 + p1;
      const uint32_t hh = pack_bf(p0, p1);
      phi[i >> 1] = hh;
      plo[i >> 1] = pack_bf(p0 - lo_bf(hh), p1 - hi_bf(hh));
    }
    psum = xor32_sum(psum);
    l_run = l_run * alpha + psum;
#pragma unroll
    for (int st = 0; st < 2; ++st) {
      pw.hi[st] = __builtin_bit_cast(bf16x8, (u32x4{phi[4 * st], phi[4 * st + 1], phi[4 * st + 2], phi[4 * st + 3]}));
      pw.lo[st] = __builtin_bit_cast(bf16x8, (u32x4{plo[4 * st], plo[4 * st + 1], plo[4 * st + 2], plo[4 * st + 3]}));
    }
    return alpha;
  };
  // O^T += V^T (P_hi + P_lo)^T for one step's V tile (16-key halves [st0, st1))
  auto pv = [&](const Pw &pw, int slot, int st0 = 0, int st1 = 2) __attribute__((always_inline)) {
    const uint8_t *vs = ring + (SL + slot) * TB;
#pragma unroll
    for (int st = st0; st < st1; ++st) {
#pragma unroll
      for (int db = 0; db < DB; ++db) {
        i16x4 hv[2];
#pragma unroll
        for (int r = 0; r < 2; ++r) {
          const int key = 32 * kh + st * 16 + 8 * r + 4 * h + (gi >> 2);
          const int d = db * 32 + 16 * (grp & 1) + 4 * (gi & 3);
          const int c = d >> 3;
          hv[r] = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (lds_i16x4 *)(vs + key * DP * 2 + 16 * (c ^ swz_v<DP>(key)) + 2 * (d & 7)));
        }
        const bf16x8 va = __builtin_bit_cast(bf16x8, __builtin_shufflevector(hv[0], hv[1], 0, 1, 2, 3, 4, 5, 6, 7));
        acc_o[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(va, pw.hi[st], acc_o[db], 0, 0, 0);
        acc_o[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(va, pw.lo[st], acc_o[db], 0, 0, 0);
      }
    }
  };
  auto rescale = [&](float alpha) __attribute__((always_inline)) {
    // alpha is 1 on the path that skips the rescale; an opaque copy keeps
    // the compiler from turning the rare branch into a multiply of the whole
    // accumulator on every step
    asm volatile("" : "+v"(alpha));
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc_o[db][e] *= alpha;
  };

  // ---- pipeline.  K tiles and V tiles live in separate rings of SL slots
  // (step t in slot t % SL of each).  Iteration s (0 <= s <= nsteps) waits
  // for K(s+1) and V(s-1), passes one barrier, refills the K slot of step s
  // (its scores were computed in iteration s-1) with K(s+SL) and the V slot
  // of step s-2 (its P V ran in iteration s-1) with V(s+SL-2), then issues
  // the K Q^T MFMAs of step s+1 and the P V MFMAs of step s-1 -- 24 MFMAs
  // that depend on nothing the softmax of step s computes -- and runs that
  // softmax on the scores of the previous iteration, so the matrix core
  // works while the VALU does.  A rescale of the accumulator waits for
  // P V(s-1), at the end of the iteration.  Steps [0, n_full) are visible
  // and unmasked for every wave of the workgroup and iterations over them
  // take a body with no per-wave branch; the others test each wave's blocks.
  using MaskT = std::integral_constant<bool, true>;
  using NoMaskT = std::integral_constant<bool, false>;
  const int lim = causal ? min(kv_end, off + q0 + 1) : kv_end;  // keys every query of the group sees
  const int n_full = max(0, min(nsteps, lim / BKV - t_begin));
  // this wave's loads: K(t) for waves 0-3 (issued SL steps ahead), V(t)
  // for waves 4-7 (SL-2 ahead); the step iteration s needs from them
  const int lead = isk ? SL : SL - 2;
  auto wait_barrier = [&](int s) __attribute__((always_inline)) {
    const int need = isk ? s + 1 : s - 1;
    const int last = min(nsteps - 1, s + lead - 1);  // newest step issued so far
    if (last - need >= SL - 2) vm_wait<(SL - 2) * NPW>();
    else vm_wait<0>();
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");  // no LDS access moves above the barrier
  };
  // islot: the slot of step s + lead, (s + lead) % SL
  auto sync = [&](int s, int islot) __attribute__((always_inline)) {
    wait_barrier(s);
    if (s + lead < nsteps) issue(s + lead, islot);
  };
  f32x16 sc{};
  Pw pw_prev;
  if (nsteps > 0) {
#pragma unroll
    for (int t = 0; t < SL; ++t)
      if (t < lead && t < nsteps) issue(t, t);
    if (isk) {
      if (nsteps - 1 >= SL - 1) vm_wait<(SL - 1) * NPW>();
      else vm_wait<0>();
    }
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    sc = qk(0);
  }
  // a general iteration: any step may be masked or invisible for this wave
  auto general = [&](int s) __attribute__((always_inline)) {
    sync(s, (s + lead) % SL);
    f32x16 nxt = sc;
    if (s + 1 < nsteps) nxt = qk((s + 1) % SL);
    if (s >= 1 && visible(s - 1)) pv(pw_prev, (s - 1) % SL);
    if (s < nsteps && visible(s)) {
      bool resc;
      const float alpha = masked(s) ? softmax(MaskT{}, s, sc, pw_prev, resc) : softmax(NoMaskT{}, s, sc, pw_prev, resc);
      if (resc) rescale(alpha);
    }
    sc = nxt;
  };
  // iterations [1, n_hot) are hot: steps s-1, s visible and unmasked for
  // every wave, step s+1 present and the step either wave type loads
  // (s + SL at most) wholly below kv_end
  const int n_whole = max(0, min(nsteps, kv_end / BKV - t_begin));
  const int n_hot = min(min(n_full, nsteps - 1), n_whole - SL);
  int s = 0;
  if (nsteps > 0) general(s++);
  // The DMA of the iteration goes out in four parts between the LDS reads of
  // the score and P V products and the softmax: issued in one burst after
  // the barrier, the loads of all 8 waves queue at the texture unit and
  // stall the waves' compute behind them.  The row max of the next step's
  // scores is taken at the end of the iteration (sc_max), where it overlaps
  // the P V products, so the next softmax starts with its exponentials
  // (config 3: 57.30 -> 57.05 us median over 40 interleaved rounds).
  float sc_max = -INFINITY;
  auto hot = [&](int s, int kslot, int vslot, int islot) __attribute__((always_inline)) {
    wait_barrier(s);
    const f32x16 nxt = qk(kslot);
    issue_rows(s + lead, islot, 0, NPW / 4);
    pv(pw_prev, vslot, 0, 1);
    issue_rows(s + lead, islot, NPW / 4, NPW / 2);
    pv(pw_prev, vslot, 1, 2);
    issue_rows(s + lead, islot, NPW / 2, 3 * NPW / 4);
    bool resc;
    const float alpha = softmax(NoMaskT{}, s, sc, pw_prev, resc, &sc_max);
    issue_rows(s + lead, islot, 3 * NPW / 4, NPW);
    if (resc) rescale(alpha);
    sc = nxt;
    sc_max = row_max(nxt);
  };
  // unrolled by SL from s = 1 (mod SL): every slot is a constant (the
  // addresses fold) and the next-step scores take turns in registers
  if (s < n_hot) sc_max = row_max(sc);
  for (; s + SL <= n_hot; s += SL) {
#pragma unroll
    for (int u = 0; u < SL; ++u) hot(s + u, (u + 2) % SL, u % SL, isk ? (u + 1) % SL : (u + SL - 1) % SL);
  }
  for (; s < n_hot; ++s) hot(s, (s + 1) % SL, (s - 1) % SL, (s + lead) % SL);
  if (nsteps > 0)
    for (; s <= nsteps; ++s) general(s);
  vm_wait<0>();
  __syncthreads();  // every wave is done with the ring

  // ---- merge the KH partial states of each query in kh order.  A lane
  // holds, for its query, 4 consecutive d in each of 16 runs: 16-byte LDS
  // writes.
  float *part = reinterpret_cast<float *>(ring) + wid * 32 * PS;
#pragma unroll
  for (int db = 0; db < DB; ++db)
#pragma unroll
    for (int j = 0; j < 4; ++j)
      *reinterpret_cast<f32x4 *>(part + (lane & 31) * PS + db * 32 + j * 8 + h * 4) =
          f32x4{acc_o[db][4 * j], acc_o[db][4 * j + 1], acc_o[db][4 * j + 2], acc_o[db][4 * j + 3]};
  if (h == 0) {
    ml_s[wid][lane & 31][0] = m_run;
    ml_s[wid][lane & 31][1] = l_run;
  }
  __syncthreads();
  // Outputs: consecutive threads own consecutive 4-float chunks of a query
  // row, so each store instruction writes whole rows.
  constexpr int CPR = DP / 4;            // chunks per row
  constexpr int RPP = FA_THREADS / CPR;  // rows per pass
  static_assert(BQ % RPP == 0, "whole passes");
  const int cc = tid % CPR, rr = tid / CPR;
  const float *mrg = reinterpret_cast<const float *>(ring);
#pragma unroll
  for (int pass = 0; pass < BQ / RPP; ++pass) {
    const int ql = pass * RPP + rr;
    const int g2 = ql >> 5, qi = ql & 31;
    const int q = q0 + ql;
    if (q >= g.S_q) break;  // later passes hold later queries
    // states are (m, l, o) with o, l relative to 2^(m c): weights 2^((m_k - M) c)
    float M = -INFINITY;
#pragma unroll
    for (int k = 0; k < KH; ++k) M = fmaxf(M, ml_s[g2 + QG * k][qi][0]);
    float wk[KH], L = 0.f;
#pragma unroll
    for (int k = 0; k < KH; ++k) {
      const float mk = ml_s[g2 + QG * k][qi][0];
      wk[k] = mk == -INFINITY ? 0.f : __builtin_amdgcn_exp2f((mk - M) * c2);
      L += ml_s[g2 + QG * k][qi][1] * wk[k];
    }
    f32x4 v = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int k = 0; k < KH; ++k)
      v += *reinterpret_cast<const f32x4 *>(mrg + (g2 + QG * k) * 32 * PS + qi * PS + 4 * cc) * wk[k];
    const size_t orow = (size_t)bh * g.S_q + q;
    if (g.splits == 1) {
      const float inv = 1.0f / L;
      *reinterpret_cast<u32x2 *>(g.O + orow * DP + 4 * cc) =
          u32x2{pack_bf(v[0] * inv, v[1] * inv), pack_bf(v[2] * inv, v[3] * inv)};
    } else {
      // this split's state for the query: max M, sum L, unnormalised o
      const size_t prow = (size_t)split * g.BH * g.S_q + orow;
      *reinterpret_cast<f32x4 *>(g.part_o + prow * DP + 4 * cc) = v;
      if (cc == 0) {
        g.part_ml[prow * 2] = M;
        g.part_ml[prow * 2 + 1] = L;
      }
    }
  }
}

// Merge of the key splits (split order), 8 outputs per thread with 16-byte
// accesses: O = sum_s o_s w_s / sum_s l_s w_s, w_s = 2^((m_s - M) c) with m
// the running max of unscaled scores and c = scale * log2(e).
template <int DP>
__device__ __forceinline__ void fa_combine_body(FaArgs g) {
  const int64_t rows = (int64_t)g.BH * g.S_q;
  const int64_t items = rows * (DP / 8);
  for (int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x; t < items; t += (int64_t)gridDim.x * 256) {
    const int64_t row = t / (DP / 8);
    const int d0 = (int)(t % (DP / 8)) * 8;
    const float c2 = g.scale * 1.4426950408889634f;
    float M = -INFINITY;
    for (int s = 0; s < g.splits; ++s) M = fmaxf(M, g.part_ml[((size_t)s * rows + row) * 2]);
    float L = 0.f;
    f32x4 a0 = {0.f, 0.f, 0.f, 0.f}, a1 = a0;
    for (int s = 0; s < g.splits; ++s) {
      const size_t pr = (size_t)s * rows + row;
      const float ms = g.part_ml[pr * 2];
      const float w = ms == -INFINITY ? 0.f : __builtin_amdgcn_exp2f((ms - M) * c2);
      L += g.part_ml[pr * 2 + 1] * w;
      a0 += *reinterpret_cast<const f32x4 *>(g.part_o + pr * DP + d0) * w;
      a1 += *reinterpret_cast<const f32x4 *>(g.part_o + pr * DP + d0 + 4) * w;
    }
    const float inv = 1.0f / L;
    const u32x4 o = {pack_bf(a0[0] * inv, a0[1] * inv), pack_bf(a0[2] * inv, a0[3] * inv),
                     pack_bf(a1[0] * inv, a1[1] * inv), pack_bf(a1[2] * inv, a1[3] * inv)};
    *reinterpret_cast<u32x4 *>(g.O + row * DP + d0) = o;
  }
}

// In-place KV append (kernels/cpu/attention.cpp:63-92 writes the concatenated
// cache out of place; here the new rows are copied behind the cached ones).
__device__ __forceinline__ void kv_append_body(pk_kv_append_args a) {
  const int64_t per = a.vec ? a.D / 8 : a.D;
  const int64_t total = a.BH * a.S_new * per;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < total; t += stride) {
    const int64_t u = t % per, rs = t / per, s = rs % a.S_new, bh = rs / a.S_new;
    const uint16_t *src = a.neu + (bh * a.S_new + s) * a.D;
    uint16_t *dst = a.cache + (bh * a.cap + a.S_cache + s) * a.D;
    if (a.vec) *reinterpret_cast<u32x4 *>(dst + u * 8) = *reinterpret_cast<const u32x4 *>(src + u * 8);
    else dst[u] = src[u];
  }
}

}  // namespace att
}  // namespace pk
