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
// Work split (attention_kernel, any D <= 256; head dims up to 1024 take
// attention_wide_kernel, which splits the dims over its waves): a workgroup = 4 waves x 32
// queries of one (b,h); K/V tiles are double-buffered in LDS.  When queries
// alone do not fill the chip the key range is split (flash-decoding style)
// and att_combine_kernel merges the fp32 partials in split order.  Head dims
// 64 and 128 with enough query tiles take attention_fa_kernel (below).
#include <cstring>

#include "attention_kernels.hpp"
#include "attention_module.hpp"

namespace pk {

namespace {

using namespace att;

// The kernels, as the library launches them (bodies in attention_kernels.hpp).
template <int DP, bool ALIGNED>
__global__ __launch_bounds__(AT_THREADS) void attention_kernel(AttArgs g) {
  att_body<DP, ALIGNED>(g);
}

template <int DP>
__global__ __launch_bounds__(256) void att_combine_kernel(AttArgs g) {
  att_combine_body<DP>(g);
}

template <bool ALIGNED>
__global__ __launch_bounds__(AW_THREADS, 1) void attention_wide_kernel(AttArgs g) {
  att_wide_body<ALIGNED>(g);
}

template <int DP, int QG, bool FUSED>
__global__ __launch_bounds__(FA_THREADS, 1) void attention_fa_kernel(FaArgs g) {
  fa_body<DP, QG, FUSED>(g);
}

template <int DP>
__global__ __launch_bounds__(256) void fa_combine_kernel(FaArgs g) {
  fa_combine_body<DP>(g);
}

__global__ __launch_bounds__(256) void kv_append_kernel(pk_kv_append_args a) { kv_append_body(a); }

// Launch an entry point of an emitted code object (hipModuleLaunchKernel),
// with the same grid and arguments the linked kernel gets.
template <typename Args>
int run_module(void *fn, const char *name, int64_t grid, int threads, Args a, hipStream_t st) {
  if (!fn) {
    set_error("attention code object has no entry point %s", name);
    return PK_ERR_UNSUPPORTED;
  }
  void *params[] = {&a};
  const hipError_t e = hipModuleLaunchKernel(static_cast<hipFunction_t>(fn), (unsigned)grid, 1, 1, threads, 1, 1, 0,
                                             st, params, nullptr);
  if (e != hipSuccess) return hip_fail(e, name);
  return PK_OK;
}

// Key splits (a power of two up to max_s, each split keeping at least
// min_steps key steps) for a grid of `tiles` workgroups: doubled only while
// the split grid still runs in one round of 256 workgroups.  Past that a split
// adds rounds, fp32 partials and the merge: 192-248 tiles split in two run as
// two rounds of half the work (config-3 shape, D 128, S_q 512, 3584 cached
// keys: 24 heads 62.7 us and 28 heads 68.6 us split in two, against 58.0 us
// for 32 heads in one unsplit round).
int split_count(int64_t tiles, int kv_steps, int min_steps, int max_s) {
  int s = 1;
  while (2 * s <= max_s && tiles * 2 * s <= 256 && kv_steps / (2 * s) >= min_steps) s *= 2;
  return s;
}

int pick_splits(int BH, int q_tiles, int kv_tiles) {
  return split_count((int64_t)BH * q_tiles, kv_tiles, 4, 1 << 20);
}

// The kernels split blockIdx.x into (bh, query tile, key split) in 32-bit
// arithmetic: the grid must stay within INT32_MAX workgroups.
int grid_ok(int64_t BH, int64_t q_tiles, int64_t splits, const char *name) {
  if (BH * q_tiles * splits <= INT32_MAX) return PK_OK;
  set_error("%s: %lld (b,h) x %lld query tiles x %lld key splits exceeds %d workgroups", name, (long long)BH,
            (long long)q_tiles, (long long)splits, INT32_MAX);
  return PK_ERR_UNSUPPORTED;
}

template <int DP>
int attention_dp(AttArgs g, hipStream_t st, const AttModule *mod) {
  const bool aligned = (g.D % 8 == 0) && aligned16(g.Q) && aligned16(g.K) && aligned16(g.V);
  g.q_tiles = (g.S_q + AT_BQ - 1) / AT_BQ;
  const int kv_tiles = (g.S_kv + AT_BKV - 1) / AT_BKV;
  g.splits = pick_splits(g.BH, g.q_tiles, kv_tiles);
  if (int rc = grid_ok(g.BH, g.q_tiles, g.splits, "attention")) return rc;
  WorkspaceLease lease;  // held until the combine kernel is queued
  if (g.splits > 1) {
    const size_t rows = (size_t)g.BH * g.S_q;
    const size_t bytes_o = (size_t)g.splits * rows * DP * sizeof(float);
    const size_t bytes = bytes_o + (size_t)g.splits * rows * 2 * sizeof(float);
    int rc = library_workspace(bytes, st, lease);
    if (rc) return rc;
    g.part_o = static_cast<float *>(lease.ptr);
    g.part_ml = reinterpret_cast<float *>(static_cast<char *>(lease.ptr) + bytes_o);
  }
  const int blocks = g.BH * g.q_tiles * g.splits;
  if (mod) {
    int rc = run_module(aligned ? mod->att : mod->att_unaligned, "pk_att", blocks, AT_THREADS, g, st);
    if (rc) return rc;
  } else {
    if (aligned) attention_kernel<DP, true><<<blocks, AT_THREADS, 0, st>>>(g);
    else attention_kernel<DP, false><<<blocks, AT_THREADS, 0, st>>>(g);
    PK_LAUNCH_CHECK("attention_kernel");
  }
  if (g.splits > 1) {
    const int64_t total = (int64_t)g.BH * g.S_q * g.D;
    const int grid = (int)std::min<int64_t>((total + 255) / 256, 8192);
    if (mod) return run_module(mod->att_combine, "pk_att_combine", grid, 256, g, st);
    att_combine_kernel<DP><<<grid, 256, 0, st>>>(g);
    PK_LAUNCH_CHECK("att_combine_kernel");
  }
  return PK_OK;
}

// Head dims 257..1024: 32 queries x 32 keys per step, 4 waves splitting the
// head dims (att_wide_body), key splits merged as for attention_dp.
int attention_wide(AttArgs g, hipStream_t st, const AttModule *mod) {
  const bool aligned = (g.D % 8 == 0) && aligned16(g.Q) && aligned16(g.K) && aligned16(g.V);
  g.q_tiles = (g.S_q + AW_BQ - 1) / AW_BQ;
  const int kv_tiles = (g.S_kv + AW_BKV - 1) / AW_BKV;
  g.splits = pick_splits(g.BH, g.q_tiles, kv_tiles);
  if (int rc = grid_ok(g.BH, g.q_tiles, g.splits, "attention")) return rc;
  WorkspaceLease lease;  // held until the combine kernel is queued
  if (g.splits > 1) {
    const size_t rows = (size_t)g.BH * g.S_q;
    const size_t bytes_o = (size_t)g.splits * rows * AW_DMAX * sizeof(float);
    const size_t bytes = bytes_o + (size_t)g.splits * rows * 2 * sizeof(float);
    int rc = library_workspace(bytes, st, lease);
    if (rc) return rc;
    g.part_o = static_cast<float *>(lease.ptr);
    g.part_ml = reinterpret_cast<float *>(static_cast<char *>(lease.ptr) + bytes_o);
  }
  const int blocks = g.BH * g.q_tiles * g.splits;
  if (mod) {
    int rc = run_module(aligned ? mod->att : mod->att_unaligned, "pk_att", blocks, AW_THREADS, g, st);
    if (rc) return rc;
  } else {
    if (aligned) attention_wide_kernel<true><<<blocks, AW_THREADS, 0, st>>>(g);
    else attention_wide_kernel<false><<<blocks, AW_THREADS, 0, st>>>(g);
    PK_LAUNCH_CHECK("attention_wide_kernel");
  }
  if (g.splits > 1) {
    const int64_t total = (int64_t)g.BH * g.S_q * g.D;
    const int grid = (int)std::min<int64_t>((total + 255) / 256, 8192);
    if (mod) return run_module(mod->att_combine, "pk_att_combine", grid, 256, g, st);
    att_combine_kernel<AW_DMAX><<<grid, 256, 0, st>>>(g);
    PK_LAUNCH_CHECK("att_combine_kernel");
  }
  return PK_OK;
}

int kv_append_inplace_launch(uint16_t *cache, const uint16_t *neu, int64_t BH, int64_t Sc, int64_t Sn, int64_t D,
                             int64_t cap, hipStream_t st, const AttModule *mod) {
  if (BH * Sn * D == 0) return PK_OK;
  const int vec = (D % 8 == 0) && aligned16(cache) && aligned16(neu);
  const int64_t units = BH * Sn * (vec ? D / 8 : D);
  const int grid = (int)std::min<int64_t>(std::max<int64_t>((units + 255) / 256, 1), 256 * 64);
  pk_kv_append_args a{cache, neu, BH, Sc, Sn, D, cap, vec};
  if (mod) return run_module(mod->kv_append, "pk_kv_append", grid, 256, a, st);
  kv_append_kernel<<<grid, 256, 0, st>>>(a);
  PK_LAUNCH_CHECK("kv_append_kernel");
  return PK_OK;
}

}  // namespace

// The flash-style kernel when the shape suits it: D 64 or 128 and 16-byte
// aligned tensors (callers also require scale > 0: the kernel tracks the
// running max on unscaled scores).  With Kn/Vn (fused append) the new rows
// must start on a key step of the tile shape (S_cache a multiple of bkv).
bool fa_applicable(int S_kv, int S_cache, int D, int kv_rows, const void *Q, const void *K, const void *V,
                   const void *O, const void *Kn, const void *Vn, const void *Kc, const void *Vc, int bkv) {
  if (D != 64 && D != 128) return false;
  if (S_kv <= 0) return false;
  if (!aligned16(Q) || !aligned16(K) || !aligned16(V) || !aligned16(O)) return false;
  if ((size_t)kv_rows * D * 2 >= (size_t(1) << 31)) return false;
  if (Kn) {
    if (!aligned16(Kn) || !aligned16(Vn) || !aligned16(Kc) || !aligned16(Vc)) return false;
    if (S_cache % bkv != 0) return false;  // one source per key step
    if ((size_t)(S_kv - S_cache) * D * 2 >= (size_t(1) << 31)) return false;
  }
  return true;
}

// The two tile shapes of the flash kernel: QG query groups of 32 and
// 8 / QG key blocks of 32 per step -- 128 queries x 64 keys (QG 4) or
// 64 queries x 128 keys (QG 2).
constexpr int fa_bq(int qg) { return 32 * qg; }
constexpr int fa_bkv(int qg) { return 32 * (FA_WAVES / qg); }

// Built-in tile shape: 128 x 64 when its query tiles alone fill the chip
// (256 workgroups); otherwise 64 x 128, which doubles the workgroups without
// the key splits (and their fp32 partials and merge kernel) that a short
// grid otherwise needs.  Causal prefills of 2048 or more queries also take
// 64 x 128: their query tiles' work grows with the tile index, and the finer
// tiles balance it (measured at D 128: S_q 2048 91.7 against 102.5 us, 4096
// 271 against 287 us, 2 x 2048 165 against 173 us; at 1024 queries 128 x 64
// wins, 35.3 against 38.4 us, and without the mask it wins at every length).
int fa_default_qg(int64_t BH, int S_q, bool causal) {
  if (causal && S_q >= 2048) return 2;
  return BH * ((S_q + fa_bq(4) - 1) / fa_bq(4)) >= 256 ? 4 : 2;
}

// Launch the flash-style kernel with QG query groups per workgroup, with
// enough key splits to reach ~256 workgroups, each split keeping >= 8 steps.
int attention_fa(FaArgs a, int D, int qg, hipStream_t st, const AttModule *mod) {
  const int BQ = fa_bq(qg), BKV = fa_bkv(qg);
  a.q_tiles = (a.S_q + BQ - 1) / BQ;
  const int ntiles = (a.S_kv + BKV - 1) / BKV;
  a.splits = split_count((int64_t)a.BH * a.q_tiles, ntiles, 8, 8);
  if (int rc = grid_ok(a.BH, a.q_tiles, a.splits, "attention")) return rc;
  WorkspaceLease lease;  // held until the merge kernel is queued
  if (a.splits > 1) {
    const size_t rows = (size_t)a.BH * a.S_q;
    const size_t bytes_o = (size_t)a.splits * rows * D * sizeof(float);
    const size_t bytes = bytes_o + (size_t)a.splits * rows * 2 * sizeof(float);
    int rc = library_workspace(bytes, st, lease);
    if (rc) return rc;
    a.part_o = static_cast<float *>(lease.ptr);
    a.part_ml = reinterpret_cast<float *>(static_cast<char *>(lease.ptr) + bytes_o);
  }
  const int blocks = a.BH * a.q_tiles * a.splits;
  const bool fused = a.Kn != nullptr;
  if (mod) {  // an emitted flash object serves the fused op only
    if (!fused) {
      set_error("attention code object: the flash entry point is the fused (append) kernel");
      return PK_ERR_UNSUPPORTED;
    }
    int rc = run_module(mod->fa_fused, "pk_fa_fused", blocks, FA_THREADS, a, st);
    if (rc || a.splits == 1) return rc;
    const int64_t items = (int64_t)a.BH * a.S_q * (D / 8);
    return run_module(mod->fa_combine, "pk_fa_combine", std::min<int64_t>((items + 255) / 256, 8192), 256, a, st);
  }
#define PK_FA_LAUNCH(DPV, QGV)                                                              \
  do {                                                                                      \
    if (fused) attention_fa_kernel<DPV, QGV, true><<<blocks, FA_THREADS, 0, st>>>(a);       \
    else attention_fa_kernel<DPV, QGV, false><<<blocks, FA_THREADS, 0, st>>>(a);            \
  } while (0)
  if (D == 128) {
    if (qg == 4) PK_FA_LAUNCH(128, 4);
    else PK_FA_LAUNCH(128, 2);
  } else {
    if (qg == 4) PK_FA_LAUNCH(64, 4);
    else PK_FA_LAUNCH(64, 2);
  }
#undef PK_FA_LAUNCH
  PK_LAUNCH_CHECK("attention_fa_kernel");
  if (a.splits > 1) {
    const int64_t items = (int64_t)a.BH * a.S_q * (D / 8);
    const int grid = (int)std::min<int64_t>((items + 255) / 256, 8192);
    if (D == 128) fa_combine_kernel<128><<<grid, 256, 0, st>>>(a);
    else fa_combine_kernel<64><<<grid, 256, 0, st>>>(a);
    PK_LAUNCH_CHECK("fa_combine_kernel");
  }
  return PK_OK;
}

// Configs of attention as descriptors: the flash kernel's two tile shapes
// for D 64 / 128 ({queries, keys per step, D, 8 waves, 16-byte vectors,
// D/16 MFMA k-steps per product, K/V ring slots}), the generic kernel
// otherwise: up to D 256 {128 queries, 64 keys, padded D, 4 waves, vector
// width, padded D / 16, 1}, above it the wide kernel {32 queries, 32 keys,
// 1024, 4 waves, vector width, 16 k-steps per wave, 1}.  unroll = MFMA
// k-steps of one query-key product (per wave for the wide kernel).
pk_config fa_config(int qg, int D) {
  return pk_config{fa_bq(qg), fa_bkv(qg), D, FA_WAVES, 8, D / 16, FA_RING / (2 * fa_bkv(qg) * D * 2)};
}
bool generic_attention_config(int D, pk_config *out) {
  if (D > 256) {
    *out = pk_config{AW_BQ, AW_BKV, AW_DMAX, AW_WAVES, D % 8 == 0 ? 8 : 1, AW_DC / 16, 1};
    return true;
  }
  const int dp = D <= 32 ? 32 : D <= 64 ? 64 : D <= 128 ? 128 : 256;
  *out = pk_config{AT_BQ, AT_BKV, dp, AT_WAVES, D % 8 == 0 ? 8 : 1, dp / 16, 1};
  return true;
}
int attention_configs(int S_q, int S_kv, int D, pk_config *out, int cap) {
  if (S_q <= 0 || S_kv <= 0 || D <= 0 || D > AW_DMAX) return 0;
  pk_config c[2];
  int n = 0;
  if (D == 64 || D == 128) {
    c[n++] = fa_config(4, D);
    c[n++] = fa_config(2, D);
  } else {
    generic_attention_config(D, &c[n++]);
  }
  for (int i = 0; i < n && i < cap; ++i) out[i] = c[i];
  return n;
}
// The built-in choice.  The shape key has no batch x heads and no mask: this
// assumes 32 (the headline configuration's and the autotuner's default) and a
// causal mask (the op is the reference's causal KV-append prefill).
bool attention_config(int S_q, int S_kv, int D, pk_config *out) {
  if (S_q <= 0 || S_kv <= 0 || D <= 0 || D > AW_DMAX) return false;
  if (D == 64 || D == 128) *out = fa_config(fa_default_qg(32, S_q, true), D);
  else generic_attention_config(D, out);
  return true;
}
// The query groups a flash config names (0: not a flash config for D).
int fa_qg_of(const pk_config &c, int D) {
  for (int qg : {4, 2}) {
    const pk_config f = fa_config(qg, D);
    if (c.block_m == f.block_m && c.block_n == f.block_n && c.block_k == f.block_k && c.num_warps == f.num_warps &&
        c.vector_width == f.vector_width && c.unroll == f.unroll && c.shared_memory_stages == f.shared_memory_stages)
      return qg;
  }
  return 0;
}

// mode 0: the built-in kernel and tile shape; 2 or 4: the flash kernel
// with that many query groups (an error when it does not apply); -1: the
// generic kernel.
int attention_run(const uint16_t *Q, const uint16_t *K, const uint16_t *V, uint16_t *O, int BH,
                  int S_q, int S_kv, int D, int kv_rows, float scale, int causal, int mode, hipStream_t st,
                  const AttModule *mod = nullptr) {
  if (mode >= 0) {
    const int qg = mode ? mode : fa_default_qg(BH, S_q, causal != 0);
    if (scale > 0.f && fa_applicable(S_kv, S_kv, D, kv_rows, Q, K, V, O, nullptr, nullptr, nullptr, nullptr,
                                     fa_bkv(qg))) {
      FaArgs a{Q, K, V, nullptr, nullptr, nullptr, nullptr, O, nullptr, nullptr, BH, S_q, S_kv, S_kv, kv_rows,
               scale, causal, 1, 1};
      return attention_fa(a, D, qg, st, mod);
    }
    if (mode) {
      set_error("attention: the flash kernel (%d x %d tiles) needs D 64 or 128, 16-byte aligned tensors and "
                "scale > 0",
                fa_bq(qg), fa_bkv(qg));
      return PK_ERR_UNSUPPORTED;
    }
  }
  AttArgs g{Q, K, V, O, nullptr, nullptr, BH, S_q, S_kv, D, kv_rows, scale, causal, 1, 1};
  if (D <= 32) return attention_dp<32>(g, st, mod);
  if (D <= 64) return attention_dp<64>(g, st, mod);
  if (D <= 128) return attention_dp<128>(g, st, mod);
  if (D <= 256) return attention_dp<256>(g, st, mod);
  if (D <= AW_DMAX) return attention_wide(g, st, mod);
  set_error("attention: head dim %d > 1024 is not supported", D);
  return PK_ERR_UNSUPPORTED;
}

int fused_kv_append_attention(const uint16_t *Q, uint16_t *Kc, uint16_t *Vc, const uint16_t *Kn,
                              const uint16_t *Vn, uint16_t *O, int B, int H, int S_q, int S_cache, int D,
                              int cache_capacity, float scale, int causal, int mode, hipStream_t st,
                              const AttModule *mod = nullptr) {
  PK_CHECK_ARG(Q && Kc && Vc && O && (S_q == 0 || (Kn && Vn)),
               "launch_fused_kv_append_attention: null tensor pointer");
  PK_CHECK_ARG(B >= 0 && H >= 0 && S_q >= 0 && S_cache >= 0 && D > 0,
               "launch_fused_kv_append_attention: invalid shape");
  PK_CHECK_ARG(cache_capacity <= INT32_MAX - 1023,
               "launch_fused_kv_append_attention: cache_capacity %d is within 1023 of INT32_MAX (the kernels round "
               "key counts up to whole tiles in 32-bit arithmetic)",
               cache_capacity);
  PK_CHECK_ARG((int64_t)S_cache + S_q <= cache_capacity,
               "launch_fused_kv_append_attention: S_cache + S_q = %lld exceeds cache_capacity %d",
               (long long)S_cache + S_q, cache_capacity);
  if (D > AW_DMAX) {  // refused before the append touches the caches
    set_error("launch_fused_kv_append_attention: head dim %d > 1024 is not supported", D);
    return PK_ERR_UNSUPPORTED;
  }
  const int64_t BH = (int64_t)B * H;
  if (BH == 0) return PK_OK;
  PK_CHECK_ARG(BH <= INT32_MAX, "launch_fused_kv_append_attention: B * H = %lld exceeds %d", (long long)BH,
               INT32_MAX);
  const int S_kv = S_cache + S_q;
  if (S_q > 0 && scale > 0.f && mode >= 0) {
    int qg = mode ? mode : fa_default_qg(BH, S_q, causal != 0);
    auto fits = [&](int g) {
      return fa_applicable(S_kv, S_cache, D, cache_capacity, Q, Kc, Vc, O, Kn, Vn, Kc, Vc, fa_bkv(g));
    };
    if (!mode && qg == 2 && !fits(2)) qg = 4;  // S_cache on a 64-key but not a 128-key step
    if (fits(qg)) {
      // the append happens inside the attention kernel
      FaArgs a{Q, Kc, Vc, Kn, Vn, Kc, Vc, O, nullptr, nullptr, (int)BH, S_q, S_kv, S_cache, cache_capacity,
               scale, causal, 1, 1};
      return attention_fa(a, D, qg, st, mod);
    }
  }
  if (mode > 0) {
    set_error("launch_fused_kv_append_attention: the flash kernel (%d x %d tiles) needs D 64 or 128, 16-byte "
              "aligned tensors, scale > 0 and S_cache a multiple of %d",
              fa_bq(mode), fa_bkv(mode), fa_bkv(mode));
    return PK_ERR_UNSUPPORTED;
  }
  int rc = kv_append_inplace_launch(Kc, Kn, BH, S_cache, S_q, D, cache_capacity, st, mod);
  if (rc) return rc;
  rc = kv_append_inplace_launch(Vc, Vn, BH, S_cache, S_q, D, cache_capacity, st, mod);
  if (rc) return rc;
  if (S_q == 0) return PK_OK;
  return attention_run(Q, Kc, Vc, O, (int)BH, S_q, S_kv, D, cache_capacity, scale, causal, mode, st, mod);
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
  PK_CHECK_ARG(S_q <= INT32_MAX - 1023 && S_kv <= INT32_MAX - 1023,
               "launch_attention_prefill: S_q = %d or S_kv = %d is within 1023 of INT32_MAX (the kernels round "
               "them up to whole tiles in 32-bit arithmetic)",
               S_q, S_kv);
  if ((int64_t)B * H * S_q == 0) return PK_OK;
  PK_CHECK_ARG((int64_t)B * H <= INT32_MAX, "launch_attention_prefill: B * H = %lld exceeds %d",
               (long long)B * H, INT32_MAX);
  return attention_run(Q, K, V, O, B * H, S_q, S_kv, D, S_kv, scale, causal, 0, (hipStream_t)stream);
}

int launch_fused_kv_append_attention(const uint16_t *Q, uint16_t *Kc, uint16_t *Vc,
                                     const uint16_t *Kn, const uint16_t *Vn, uint16_t *O, int B,
                                     int H, int S_q, int S_cache, int D, int cache_capacity,
                                     float scale, int causal, void *stream) {
  return fused_kv_append_attention(Q, Kc, Vc, Kn, Vn, O, B, H, S_q, S_cache, D, cache_capacity, scale, causal, 0,
                                   (hipStream_t)stream);
}

int pk_fused_kv_append_attention_config(const uint16_t *Q, uint16_t *Kc, uint16_t *Vc, const uint16_t *Kn,
                                        const uint16_t *Vn, uint16_t *O, int B, int H, int S_q, int S_cache,
                                        int D, int cache_capacity, float scale, int causal, const pk_config *cfg,
                                        void *stream) {
  return fused_kv_append_attention_module(Q, Kc, Vc, Kn, Vn, O, B, H, S_q, S_cache, D, cache_capacity, scale,
                                          causal, cfg, nullptr, stream);
}

}  // extern "C"

namespace pk {

int fused_kv_append_attention_module(const uint16_t *Q, uint16_t *Kc, uint16_t *Vc, const uint16_t *Kn,
                                     const uint16_t *Vn, uint16_t *O, int B, int H, int S_q, int S_cache, int D,
                                     int cache_capacity, float scale, int causal, const pk_config *cfg,
                                     const AttModule *mod, void *stream) {
  int mode = 0;
  if (cfg) {
    pk_config gen{};
    generic_attention_config(D, &gen);
    mode = fa_qg_of(*cfg, D);
    if (!mode) {
      PK_CHECK_ARG(std::memcmp(cfg, &gen, sizeof gen) == 0,
                   "pk_fused_kv_append_attention_config: {%d, %d, %d, %d, %d, %d, %d} is not a config of the "
                   "gfx950 attention kernels for D = %d",
                   cfg->block_m, cfg->block_n, cfg->block_k, cfg->num_warps, cfg->vector_width, cfg->unroll,
                   cfg->shared_memory_stages, D);
      mode = -1;
    }
  }
  PK_CHECK_ARG(!mod || cfg, "fused_kv_append_attention: a code object needs its config");
  return fused_kv_append_attention(Q, Kc, Vc, Kn, Vn, O, B, H, S_q, S_cache, D, cache_capacity, scale, causal,
                                   mode, (hipStream_t)stream, mod);
}

}  // namespace pk
