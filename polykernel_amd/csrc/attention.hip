// attention.hip -- causal prefill attention with KV append for gfx950.
//
// Arithmetic of kernels/cpu/attention.cpp:95-163: for query i of a (b,h) the
// visible keys are j <= S_kv - S_q + i (causal) or all j; score = (q.k) * scale
// in fp32; softmax in fp32; o = bf16(sum_j p_j v_j / sum_j p_j).  Here the
// softmax is computed online over 64-key tiles (running max / sum, fp32) and
// both products run on v_mfma_f32_32x32x16_bf16 with fp32 accumulation.  The
// reference keeps the softmax weights in fp32; here each weight is split into
// two bf16 halves (p = p_hi + p_lo) and the PV product is two MFMAs, so the
// weights reach the product to ~2^-17 relative, and the row sum uses the fp32
// weights -- leaving summation order and exp() rounding as the differences.
//
// Layout trick: the kernel computes S^T = K Q^T, so in the accumulator each
// lane owns one query (lane % 32) and 16 keys; the per-query max/sum need one
// xor-32 shuffle.  The PV product is computed transposed as O^T = V^T P^T:
// the B operand is the P^T accumulator itself (its 8 k-slots are the keys
// [4h..4h+3, 8+4h..8+4h+3] of a 16-key step, h = lane / 32) and the A operand
// V^T is assembled from the V tile in LDS by ds_read_b64_tr_b16 in exactly
// that key order, so P never leaves registers and the rescale by
// exp(m_old - m_new) is a per-lane multiply.
//
// Work split: a workgroup = 4 waves x 32 queries of one (b,h); K/V tiles are
// double-buffered in LDS.  When queries alone do not fill the chip the key
// range is split (flash-decoding style) and att_combine_kernel merges the
// fp32 partials in split order.
#include "pk_common.hpp"

namespace pk {

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) i16x4 lds_i16x4;

constexpr int AT_WAVES = 4;
constexpr int AT_BQ = AT_WAVES * 32;
constexpr int AT_BKV = 64;
constexpr int AT_THREADS = AT_WAVES * 64;

struct AttArgs {
  const uint16_t *Q, *K, *V;
  uint16_t *O;
  float *part_o;  // [splits][BH][S_q][DP] when splits > 1
  float *part_ml; // [splits][BH][S_q][2]
  int BH, S_q, S_kv, D;
  int kv_rows;    // rows per (b,h) in K/V storage (>= S_kv)
  float scale;
  int causal;
  int splits;
  int q_tiles;
};

// V rows: 16-byte-chunk XOR so the 4 rows of one 16-lane transpose read hit
// distinct banks (rows of 64 B pair up in one 128-byte bank sweep when DP = 32).
template <int DP>
__device__ __forceinline__ int swz_v(int k) {
  if constexpr (DP >= 128) {
    constexpr int t[4] = {0, 4, 10, 14};
    return t[k & 3];
  } else if constexpr (DP == 64) {
    return (k & 3) * 2;
  } else {
    return ((k >> 1) & 1) * 2;
  }
}

// K rows: XOR the chunk index with the row inside aligned groups of 8 chunks
// (4 when a row has only 4 chunks) for conflict-free ds_read_b128.
template <int CH>
__device__ __forceinline__ int swz_k(int c, int row) {
  if constexpr (CH >= 8) return (c & ~7) | ((c & 7) ^ (row & 7));
  else return c ^ (row & 3);
}

template <int DP, bool ALIGNED>
__global__ __launch_bounds__(AT_THREADS) void attention_kernel(AttArgs g) {
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
  for (int t = t_begin; t < t_end; ++t) {
    const int cur = (t - t_begin) & 1;
    if (t + 1 < t_end) load_kv(t + 1);
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
    tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
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
    psum += __shfl_xor(psum, 32, 64);
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

template <int DP>
__global__ __launch_bounds__(256) void att_combine_kernel(AttArgs g) {
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

int pick_splits(int BH, int q_tiles, int kv_tiles) {
  int s = 1;
  while (BH * q_tiles * s < 256 && kv_tiles / (2 * s) >= 4) s *= 2;
  return s;
}

template <int DP>
int attention_dp(AttArgs g, hipStream_t st) {
  const bool aligned = (g.D % 8 == 0) && aligned16(g.Q) && aligned16(g.K) && aligned16(g.V);
  g.q_tiles = (g.S_q + AT_BQ - 1) / AT_BQ;
  const int kv_tiles = (g.S_kv + AT_BKV - 1) / AT_BKV;
  g.splits = pick_splits(g.BH, g.q_tiles, kv_tiles);
  if (g.splits > 1) {
    const size_t rows = (size_t)g.BH * g.S_q;
    const size_t bytes_o = (size_t)g.splits * rows * DP * sizeof(float);
    const size_t bytes = bytes_o + (size_t)g.splits * rows * 2 * sizeof(float);
    void *ws = nullptr;
    int rc = library_workspace(bytes, &ws);
    if (rc) return rc;
    g.part_o = static_cast<float *>(ws);
    g.part_ml = reinterpret_cast<float *>(static_cast<char *>(ws) + bytes_o);
  }
  const int blocks = g.BH * g.q_tiles * g.splits;
  if (aligned) attention_kernel<DP, true><<<blocks, AT_THREADS, 0, st>>>(g);
  else attention_kernel<DP, false><<<blocks, AT_THREADS, 0, st>>>(g);
  PK_LAUNCH_CHECK("attention_kernel");
  if (g.splits > 1) {
    const int64_t total = (int64_t)g.BH * g.S_q * g.D;
    att_combine_kernel<DP><<<(int)std::min<int64_t>((total + 255) / 256, 8192), 256, 0, st>>>(g);
    PK_LAUNCH_CHECK("att_combine_kernel");
  }
  return PK_OK;
}

}  // namespace

int kv_append_inplace_launch(uint16_t *cache, const uint16_t *neu, int64_t BH, int64_t Sc,
                             int64_t Sn, int64_t D, int64_t cap, hipStream_t st);

int attention_run(const uint16_t *Q, const uint16_t *K, const uint16_t *V, uint16_t *O, int BH,
                  int S_q, int S_kv, int D, int kv_rows, float scale, int causal, hipStream_t st) {
  AttArgs g{Q, K, V, O, nullptr, nullptr, BH, S_q, S_kv, D, kv_rows, scale, causal, 1, 1};
  if (D <= 32) return attention_dp<32>(g, st);
  if (D <= 64) return attention_dp<64>(g, st);
  if (D <= 128) return attention_dp<128>(g, st);
  set_error("attention: head dim %d > 128 is not supported", D);
  return PK_ERR_UNSUPPORTED;
}

}  // namespace pk

using namespace pk;

extern "C" {

int launch_attention_prefill(const uint16_t *Q, const uint16_t *K, const uint16_t *V, uint16_t *O,
                             int B, int H, int S_q, int S_kv, int D, float scale, int causal,
                             void *stream) {
  PK_CHECK_ARG(Q && K && V && O, "launch_attention_prefill: null tensor pointer");
  PK_CHECK_ARG(B >= 0 && H >= 0 && S_q >= 0 && S_kv >= 0 && D > 0,
               "launch_attention_prefill: invalid shape");
  if ((int64_t)B * H * S_q == 0) return PK_OK;
  return attention_run(Q, K, V, O, B * H, S_q, S_kv, D, S_kv, scale, causal, (hipStream_t)stream);
}

int launch_fused_kv_append_attention(const uint16_t *Q, uint16_t *Kc, uint16_t *Vc,
                                     const uint16_t *Kn, const uint16_t *Vn, uint16_t *O, int B,
                                     int H, int S_q, int S_cache, int D, int cache_capacity,
                                     float scale, int causal, void *stream) {
  PK_CHECK_ARG(Q && Kc && Vc && O && (S_q == 0 || (Kn && Vn)),
               "launch_fused_kv_append_attention: null tensor pointer");
  PK_CHECK_ARG(B >= 0 && H >= 0 && S_q >= 0 && S_cache >= 0 && D > 0,
               "launch_fused_kv_append_attention: invalid shape");
  PK_CHECK_ARG((int64_t)S_cache + S_q <= cache_capacity,
               "launch_fused_kv_append_attention: S_cache + S_q = %lld exceeds cache_capacity %d",
               (long long)S_cache + S_q, cache_capacity);
  hipStream_t st = (hipStream_t)stream;
  const int64_t BH = (int64_t)B * H;
  if (BH == 0) return PK_OK;
  int rc = kv_append_inplace_launch(Kc, Kn, BH, S_cache, S_q, D, cache_capacity, st);
  if (rc) return rc;
  rc = kv_append_inplace_launch(Vc, Vn, BH, S_cache, S_q, D, cache_capacity, st);
  if (rc) return rc;
  if (S_q == 0) return PK_OK;
  return attention_run(Q, Kc, Vc, O, (int)BH, S_q, S_cache + S_q, D, cache_capacity, scale, causal, st);
}

}  // extern "C"
