// int8.hip -- int8 weight-only matmul for decode shapes (small M) on gfx950.
//
// C[M,N] = bf16(scale[n] * sum_k A[m,k] * Wq[k,n]), A bf16 [M,K], Wq int8 [K,N]
// (N contiguous, the reference layout of kernels/generated/matmul_int8.cu:47-88).
// The per-channel scale is applied once to the fp32 dot product instead of to
// every weight (kernels/cpu/matmul_quant.cpp:189-199 dequantises per element);
// int8 values and their products with bf16 activations are exact in fp32, so
// only the summation order and that one rounding differ.
//
// Streaming design (HBM-bound: every weight byte is read once):
//   - a workgroup owns a 64-column slice of N and a K range (split-K);
//   - each of its 4 waves streams a quarter of that K range in 32-row steps:
//     two 16-byte loads per lane fetch a 32x64 int8 block, which is widened to
//     bf16 in registers (exact) and written to the wave's private LDS block in
//     the swizzled N-contiguous layout of the bf16 GEMM;
//   - ds_read_b64_tr_b16 assembles the MFMA B operand (8 consecutive k of one
//     column); A (16 rows of activations) is read straight from global/L2;
//   - v_mfma_f32_16x16x32_bf16, 4 column blocks per step;
//   - the 4 waves' accumulators are summed in LDS in a fixed order; with one
//     K split the epilogue runs in place, otherwise fp32 partials go to a
//     workspace and int8_reduce_kernel sums the splits in split order.
// Epilogues: plain, GELU (exact table) and residual add, each with the
// golden's per-stage bf16 rounding.
#include <mutex>

#include "int8_stream.hpp"

namespace pk {

namespace {

using namespace i8s;

constexpr int I8_BN = 64;      // columns per workgroup
constexpr int I8_STEP = 32;    // k rows per wave step
constexpr int I8_WAVES = 4;
constexpr int I8_THREADS = I8_WAVES * 64;

struct Int8Args {
  const uint16_t *A;
  const int8_t *W;
  const float *scale;
  float *partial;  // [splits][M][N] when splits > 1
  uint16_t *C;
  const uint16_t *R;
  const uint16_t *gelu_tab;
  int M, N, K;
  int splits;
  int kper;  // rows of K per split (multiple of I8_STEP * I8_WAVES)
};

__device__ __forceinline__ int swz64(int k) { return (k & 3) * 2; }

// Widen 4 int8 (one dword) to 4 bf16 in two dwords.  int8 -> fp32 is exact and
// the fp32 value has at most 8 significant bits, so its top half is the bf16.
__device__ __forceinline__ void widen4(uint32_t w, uint32_t &lo, uint32_t &hi) {
  const float f0 = (float)(int8_t)(w & 0xFF), f1 = (float)(int8_t)((w >> 8) & 0xFF);
  const float f2 = (float)(int8_t)((w >> 16) & 0xFF), f3 = (float)(int8_t)(w >> 24);
  lo = (__float_as_uint(f0) >> 16) | (__float_as_uint(f1) & 0xFFFF0000u);
  hi = (__float_as_uint(f2) >> 16) | (__float_as_uint(f3) & 0xFFFF0000u);
}

template <int EPI>
__device__ __forceinline__ uint16_t int8_epilogue(float dot, int m, int n, const Int8Args &g) {
#pragma clang fp contract(off)
  const uint32_t t = f2bf(dot * g.scale[n]);
  if constexpr (EPI == I8_NONE) {
    return (uint16_t)t;
  } else if constexpr (EPI == I8_GELU) {
    return (uint16_t)gelu_bits(t, g.gelu_tab);
  } else {
    return (uint16_t)f2bf(bf2f(t) + bf2f(g.R[(size_t)m * g.N + n]));
  }
}

template <bool ALIGNED, int EPI>
__global__ __launch_bounds__(I8_THREADS) void int8_gemm_kernel(Int8Args g) {
  __shared__ __attribute__((aligned(16))) uint16_t wlds[I8_WAVES][I8_STEP * I8_BN];
  __shared__ float red[I8_WAVES][16 * I8_BN];

  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int n0 = blockIdx.x * I8_BN;
  const int split = blockIdx.y;
  const int m0 = blockIdx.z * 16;
  const int kb0 = split * g.kper;
  const int kb1 = min(g.K, kb0 + g.kper);
  const int wk = g.kper / I8_WAVES;  // rows per wave
  const int kw0 = kb0 + wid * wk;
  const int kw1 = min(kb1, kw0 + wk);

  uint16_t *my = wlds[wid];
  f32x4 acc[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};

  // A operand (16x16x32): row m = lane % 16, k = 8 * (lane / 16) + 0..7.
  const int am = m0 + (lane & 15);
  const int ak = 8 * (lane >> 4);
  // W block loads: part p covers rows p*16 + lane/4, columns (lane%4)*16 .. +15.
  const int wr = lane >> 2, wc = (lane & 3) * 16;
  // tr-read coordinates (per 16-lane group g: k base 8g; lane i -> row i/4, col 4*(i%4)).
  const int grp = lane >> 4, gi = lane & 15;

  for (int k0 = kw0; k0 < kw1; k0 += I8_STEP) {
    // ---- loads
    u32x4 wv[2];
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      const int k = k0 + p * 16 + wr;
      const int n = n0 + wc;
      if constexpr (ALIGNED) {
        wv[p] = (k < kw1 && n < g.N) ? *reinterpret_cast<const u32x4 *>(g.W + (size_t)k * g.N + n)
                                     : u32x4{0, 0, 0, 0};
      } else {
        uint32_t w4[4] = {0, 0, 0, 0};
        if (k < kw1) {
#pragma unroll
          for (int e = 0; e < 16; ++e)
            if (n + e < g.N)
              w4[e >> 2] |= ((uint32_t)(uint8_t)g.W[(size_t)k * g.N + n + e]) << (8 * (e & 3));
        }
        wv[p] = u32x4{w4[0], w4[1], w4[2], w4[3]};
      }
    }
    u32x4 av;
    {
      const int k = k0 + ak;
      if constexpr (ALIGNED) {
        av = (am < g.M && k < kw1) ? *reinterpret_cast<const u32x4 *>(g.A + (size_t)am * g.K + k)
                                   : u32x4{0, 0, 0, 0};
      } else {
        uint32_t a4[4] = {0, 0, 0, 0};
        if (am < g.M) {
#pragma unroll
          for (int e = 0; e < 8; ++e)
            if (k + e < kw1) a4[e >> 1] |= (uint32_t)g.A[(size_t)am * g.K + k + e] << (16 * (e & 1));
        }
        av = u32x4{a4[0], a4[1], a4[2], a4[3]};
      }
    }
    // ---- widen to bf16 and stage in this wave's LDS block
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      const int row = p * 16 + wr;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        uint32_t o0, o1, o2, o3;
        widen4(wv[p][2 * h], o0, o1);
        widen4(wv[p][2 * h + 1], o2, o3);
        const u32x4 o = {o0, o1, o2, o3};
        const int c = (wc >> 3) + h;  // 16-byte chunk of the 128-byte row
        *reinterpret_cast<u32x4 *>(my + row * I8_BN + ((c ^ swz64(row)) << 3)) = o;
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const bf16x8 a = __builtin_bit_cast(bf16x8, av);
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) {
      i16x4 h[2];
#pragma unroll
      for (int r = 0; r < 2; ++r) {
        const int row = 8 * grp + 4 * r + (gi >> 2);
        const int col = nb * 16 + 4 * (gi & 3);
        const int c = col >> 3;
        h[r] = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (lds_i16x4 *)(my + row * I8_BN + ((c ^ swz64(row)) << 3) + (col & 7)));
      }
      short tmp[8] = {h[0][0], h[0][1], h[0][2], h[0][3], h[1][0], h[1][1], h[1][2], h[1][3]};
      acc[nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, __builtin_bit_cast(bf16x8, tmp), acc[nb],
                                                        0, 0, 0);
    }
    // The next step overwrites this wave's block: keep its reads ahead of those writes.
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }

  // ---- cross-wave reduction (fixed order) -> epilogue or partial
  // D layout (16x16): acc[nb][i] -> row (lane/16)*4 + i, col nb*16 + lane%16.
#pragma unroll
  for (int nb = 0; nb < 4; ++nb)
#pragma unroll
    for (int i = 0; i < 4; ++i) red[wid][((lane >> 4) * 4 + i) * I8_BN + nb * 16 + (lane & 15)] = acc[nb][i];
  __syncthreads();
  for (int e = tid; e < 16 * I8_BN; e += I8_THREADS) {
    const int r = e / I8_BN, c = e % I8_BN;
    const int m = m0 + r, n = n0 + c;
    if (m >= g.M || n >= g.N) continue;
    float s = red[0][e];
#pragma unroll
    for (int w = 1; w < I8_WAVES; ++w) s += red[w][e];
    if (g.splits > 1)
      g.partial[((size_t)split * g.M + m) * g.N + n] = s;
    else
      g.C[(size_t)m * g.N + n] = int8_epilogue<EPI>(s, m, n, g);
  }
}

// Split reduction, 8 outputs per thread: the partials of all splits are
// loaded with 16-byte loads (independent, so they are all in flight at once)
// and added in split order.  Needs N % 8 == 0 and 16-byte aligned buffers.
template <int EPI>
__global__ __launch_bounds__(PK_I8_REDUCE_THREADS) void int8_reduce8_kernel(Int8Args g) {
  reduce8_body<EPI>(g.partial, g.splits, g.M, g.N, g.scale, g.R, g.gelu_tab, g.C);
}

template <int EPI>
__global__ __launch_bounds__(256) void int8_reduce_kernel(Int8Args g) {
  const int64_t total = (int64_t)g.M * g.N;
  for (int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x; t < total; t += (int64_t)gridDim.x * 256) {
    float s = g.partial[t];
    for (int sp = 1; sp < g.splits; ++sp) s += g.partial[(size_t)sp * total + t];
    const int m = (int)(t / g.N), n = (int)(t % g.N);
    g.C[t] = int8_epilogue<EPI>(s, m, n, g);
  }
}

// The streaming kernel (body in int8_stream.hpp, shared with emitted code
// objects).
template <int NT, int MT, int WAVES, int STAGES, int EPI>
__global__ __launch_bounds__(WAVES * 64, 1) void int8_stream_kernel(I8sArgs g) {
  stream_body<NT, MT, WAVES, STAGES, EPI>(g);
}

// Number of K splits: enough workgroups to cover the chip ~4x, each wave
// keeping at least 8 steps.
int choose_splits(int M, int N, int K) {
  const int tiles = ((N + I8_BN - 1) / I8_BN) * ((M + 15) / 16);
  const int unit = I8_STEP * I8_WAVES;
  const int kunits = (K + unit - 1) / unit;
  int s = 1;
  while (tiles * s < 1024 && kunits / (2 * s) >= 2) s *= 2;
  return s;
}

// ---- streaming-kernel variants and their selection -------------------------
template <int NT, int MT, int WAVES, int STAGES, int EPI>
void i8s_launch(dim3 grid, hipStream_t st, const I8sArgs &g) {
  int8_stream_kernel<NT, MT, WAVES, STAGES, EPI><<<grid, WAVES * 64, 0, st>>>(g);
}
using I8sLaunch = void (*)(dim3, hipStream_t, const I8sArgs &);
struct I8sVariant {
  int nt, mt, waves, stages;
  I8sLaunch fn[3];
};
#define I8S_V(NT, MT, W, S)                                                                  \
  {                                                                                         \
    NT, MT, W, S, {                                                                         \
      i8s_launch<NT, MT, W, S, I8_NONE>, i8s_launch<NT, MT, W, S, I8_GELU>,                 \
          i8s_launch<NT, MT, W, S, I8_RESID>                                                \
    }                                                                                       \
  }
// (NT, MT, WAVES, STAGES): a workgroup covers 16*NT*WAVES columns.  LDS per
// workgroup: stages * waves * 1 KiB * (NT + 2 MT) <= 144 KiB.  In order of
// preference among equal-cost choices.
const I8sVariant kI8s[] = {
    I8S_V(8, 1, 4, 3), I8S_V(7, 1, 4, 3), I8S_V(8, 1, 2, 6), I8S_V(4, 1, 4, 6), I8S_V(4, 1, 8, 3),
    I8S_V(16, 1, 2, 4), I8S_V(2, 1, 4, 6), I8S_V(1, 1, 4, 6), I8S_V(7, 1, 4, 4),
    I8S_V(8, 2, 4, 3), I8S_V(4, 2, 4, 4), I8S_V(2, 2, 4, 6),
    I8S_V(8, 4, 4, 2), I8S_V(4, 4, 4, 3), I8S_V(2, 4, 4, 3),
};
#undef I8S_V

int device_cus() {
  static int cached[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (!cached[dev]) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      n = 256;
    cached[dev] = n;
  }
  return cached[dev];
}

struct I8sPlan {
  const I8sVariant *v = nullptr;
  int splits = 1, split_steps = 0, slices = 0, mblocks = 0;
};

bool i8s_shape_ok(int M, int N, int K) {
  return M > 0 && N > 0 && K > 0 && N % 16 == 0 && K % I8S_KSTEP == 0 && (size_t)K * N < (size_t(1) << 31) &&
         (size_t)M * K * 2 < (size_t(1) << 31);
}

// Relative streaming rate of a workgroup of `waves` waves that reads `run`
// contiguous bytes per weight row, from measurements on MI355X with rotating
// 256 MiB buffers: 512 B runs of 4 waves ~5.0 TB/s (the contiguous-read
// ceiling is ~5.7), 128 B ~3.4; 256 B runs probed at ~4.4 but the kernel
// itself streams them at 0.77-0.8 of its 512 B rate (M 16: [4096, 11008]
// 20.1 us with 256-column units against 16.7 with 512, equal bytes per unit);
// runs that are not a multiple of the 128 B cache line lose ~15 % (lines
// shared by two CUs); 2 or 8 waves per workgroup lose ~10 %.
double i8s_run_efficiency(int run, int waves) {
  double e = run >= 512 ? 1.0 : run >= 256 ? 0.8 : run >= 128 ? 0.68 : run >= 64 ? 0.55 : 0.4;
  if (run % 128 != 0) e *= 0.85;
  if (waves != 4) e *= 0.9;
  return e;
}

// Pick the variant and K split for a shape: every CU should stream the same
// number of weight bytes once (units = slices * splits * m-blocks, close to a
// multiple of the usable CU count), in runs of >= 256 B per row; splits cost
// their fp32 partials (written and read back) plus a second launch (counted
// as ~24 MB of HBM time).  Rounds are counted against 7/8 of the CUs: with
// one unit per CU the launch behaves like two rounds (measured at M 16, 512
// columns per unit: [8192, 8192] 23.9 us at 256 units, 23.5 at 304, 17.6 at
// 192; [4096, 16384] 22.4 at 256, 19.5 at 208; [16384, 4096] 22.7 at 256,
// 19.9 at 160), while 220-224 units stream at full rate.  Fields of `req`
// that are nonzero are honoured; returns false when nothing matches.
bool i8s_plan(int M, int N, int K, const pk_config *req, int cus, I8sPlan &best) {
  if (!i8s_shape_ok(M, N, K)) return false;
  const int ksteps = K / I8S_KSTEP;
  // rows per block: 16 up to M 16, 32 up to M 64 (two blocks at M 64: the
  // 64-row variant holds only two ring stages; measured M 64 [8192, 28672]
  // 66.1 against 71.3 us, [4096, 14336] 28.6 against 31.2), 64 above.  At
  // M 32 two 16-row blocks lose once the weights outgrow the MALL (the
  // second block re-reads them from HBM: [28672, 8192] 60.8 against 48.7 us),
  // so they are taken only for weights of at most 128 MiB (half the MALL:
  // [14336, 4096] 22.9 against 25.2 us, [4096, 14336] 23.4 against 26.5)
  int mt = M <= 16 ? 1 : M <= 64 ? 2 : 4;
  if (M <= 32 && (size_t)K * N <= (size_t(128) << 20)) mt = 1;
  if (req && req->block_m) {
    if (req->block_m != 16 && req->block_m != 32 && req->block_m != 64) return false;
    mt = req->block_m / 16;
  }
  if (req && req->block_k && (req->block_k % I8S_KSTEP != 0 || req->block_k <= 0)) return false;
  if (req && req->vector_width && req->vector_width != I8S_VECTOR_WIDTH) return false;
  if (req && req->unroll && req->unroll != I8S_UNROLL) return false;
  double best_cost = 0;
  bool found = false;
  for (const I8sVariant &v : kI8s) {
    const int nb = 16 * v.nt * v.waves;  // columns per workgroup
    if (v.mt != mt) continue;
    if (req && req->block_n && req->block_n != nb) continue;
    if (req && req->num_warps && req->num_warps != v.waves) continue;
    if (req && req->shared_memory_stages && req->shared_memory_stages != v.stages) continue;
    const int slices = (N + nb - 1) / nb;
    const int mblocks = (M + 16 * mt - 1) / (16 * mt);
    static const int kSplits[] = {1, 2, 3, 4, 5, 6, 7, 8, 10, 12, 14, 16, 20, 24, 28, 32};
    for (int s_req : kSplits) {
      int split_steps;
      if (req && req->block_k) {
        if (s_req != 1) break;
        split_steps = std::min(ksteps, req->block_k / I8S_KSTEP);
      } else {
        split_steps = (ksteps + s_req - 1) / s_req;
        if (s_req > 1 && split_steps < 4) break;
      }
      const int splits = (ksteps + split_steps - 1) / split_steps;
      const double units = (double)slices * splits * mblocks;
      const double rounds = std::ceil(units / std::max(1, cus * 7 / 8));
      const int run = std::min(nb, N);
      double cost = rounds * split_steps * I8S_KSTEP * (double)run * cus / i8s_run_efficiency(run, v.waves);
      if (splits > 1) cost += 2.0 * splits * M * (double)N * 4 + 24e6;
      if (!found || cost < best_cost * (1 - 1e-9)) {
        found = true;
        best_cost = cost;
        best.v = &v;
        best.splits = splits;
        best.split_steps = split_steps;
        best.slices = slices;
        best.mblocks = mblocks;
      }
    }
  }
  return found;
}

size_t i8s_workspace(const I8sPlan &p, int M, int N) {
  return p.splits > 1 ? (size_t)p.splits * M * N * sizeof(float) : 0;
}

pk_config i8s_config(const I8sVariant &v, int split_steps) {
  return pk_config{16 * v.mt, 16 * v.nt * v.waves, split_steps * I8S_KSTEP, v.waves,
                   I8S_VECTOR_WIDTH, I8S_UNROLL, v.stages};
}

}  // namespace

// Every (variant, K split) the streaming kernel offers for the shape: row
// blocks of 16, 32 or 64 up to M, each variant at every distinct split of
// >= 4 ring steps per workgroup (as i8s_plan searches them).
int int8_configs(int M, int N, int K, pk_config *out, int cap) {
  if (M <= 0 || N <= 0 || K <= 0 || !i8s_shape_ok(M, N, K)) return 0;
  const int ksteps = K / I8S_KSTEP;
  const int mt_max = M <= 16 ? 1 : M <= 32 ? 2 : 4;
  int n = 0;
  for (const I8sVariant &v : kI8s) {
    if (v.mt > mt_max) continue;
    int last = -1;
    static const int kSplits[] = {1, 2, 3, 4, 5, 6, 7, 8, 10, 12, 14, 16, 20, 24, 28, 32};
    for (int s : kSplits) {
      const int split_steps = (ksteps + s - 1) / s;
      if (s > 1 && split_steps < 4) break;
      if (split_steps == last) continue;
      last = split_steps;
      if (n < cap && out) out[n] = i8s_config(v, split_steps);
      ++n;
    }
  }
  return n;
}

bool int8_default(int M, int N, int K, pk_config *out) {
  I8sPlan p;
  if (!i8s_plan(M, N, K, nullptr, device_cus(), p)) return false;
  *out = i8s_config(*p.v, p.split_steps);
  return true;
}

// Workspace for the built-in choice, whichever kernel the pointers' alignment
// leads to.
size_t int8_workspace_bytes(int M, int N, int K) {
  if (M <= 0 || N <= 0 || K <= 0) return 0;
  size_t need = 0;
  I8sPlan p;
  if (i8s_plan(M, N, K, nullptr, device_cus(), p)) need = i8s_workspace(p, M, N);
  const int s = choose_splits(M, N, K);
  return std::max(need, s > 1 ? (size_t)s * M * N * sizeof(float) : 0);
}

static int use_workspace(size_t need, void *&ws, size_t ws_bytes, hipStream_t st, WorkspaceLease &lease) {
  if (need == 0) return PK_OK;
  if (ws == nullptr) {
    int rc = library_workspace(need, st, lease);
    ws = lease.ptr;
    return rc;
  }
  if (ws_bytes < need) {
    set_error("int8 matmul: workspace of %zu bytes required, got %zu", need, ws_bytes);
    return PK_ERR_WORKSPACE;
  }
  return PK_OK;
}

int int8_run(int epi, const uint16_t *A, const int8_t *W, const float *scale, uint16_t *C,
             const uint16_t *R, int M, int N, int K, const pk_config *cfg, void *ws,
             size_t ws_bytes, hipStream_t st) {
  const uint16_t *tab = nullptr;
  if (epi == I8_GELU) {
    int rc = gelu_table(&tab);
    if (rc) return rc;
  }
  I8sPlan plan;
  const bool fast = aligned16(A) && aligned16(W) && aligned16(scale) && aligned16(C) &&
                    (epi != I8_RESID || aligned16(R)) && i8s_plan(M, N, K, cfg, device_cus(), plan);
  if (cfg && !fast) {
    set_error("int8 matmul: configuration {block_m %d, block_n %d, block_k %d, num_warps %d, "
              "vector_width %d, unroll %d, stages %d} not available for M=%d N=%d K=%d%s",
              cfg->block_m, cfg->block_n, cfg->block_k, cfg->num_warps, cfg->vector_width, cfg->unroll,
              cfg->shared_memory_stages, M, N, K,
              i8s_shape_ok(M, N, K) ? "" : " (the shape or operand alignment needs the generic kernel)");
    return PK_ERR_UNSUPPORTED;
  }
  Int8Args g{A, W, scale, nullptr, C, R, tab, M, N, K, 1, 0};
  WorkspaceLease lease;  // library scratch, held until the reduction is queued
  if (fast) {
    int rc = use_workspace(i8s_workspace(plan, M, N), ws, ws_bytes, st, lease);
    if (rc) return rc;
    if (plan.splits > 1 && !aligned16(ws)) {
      set_error("int8 matmul: workspace must be 16-byte aligned");
      return PK_ERR_WORKSPACE;
    }
    I8sArgs a{A, W, scale, static_cast<float *>(ws), C, R, tab, M, N, K,
              plan.splits, plan.split_steps, plan.slices * plan.splits};
    plan.v->fn[epi](dim3(plan.slices * plan.splits, plan.mblocks), st, a);
    PK_LAUNCH_CHECK("int8_stream_kernel");
    g.splits = plan.splits;
    g.partial = a.partial;
  } else {
    g.splits = choose_splits(M, N, K);
    const int unit = I8_STEP * I8_WAVES;
    g.kper = ((K + g.splits - 1) / g.splits + unit - 1) / unit * unit;
    g.splits = (K + g.kper - 1) / g.kper;
    int rc = use_workspace(g.splits > 1 ? (size_t)g.splits * M * N * sizeof(float) : 0, ws, ws_bytes, st, lease);
    if (rc) return rc;
    g.partial = static_cast<float *>(ws);
    const bool aligned = (N % 16 == 0) && (K % 8 == 0) && aligned16(A) && aligned16(W);
    dim3 grid((N + I8_BN - 1) / I8_BN, g.splits, (M + 15) / 16);
#define PK_I8(E)                                                                          \
  do {                                                                                    \
    if (aligned) int8_gemm_kernel<true, E><<<grid, I8_THREADS, 0, st>>>(g);               \
    else int8_gemm_kernel<false, E><<<grid, I8_THREADS, 0, st>>>(g);                      \
  } while (0)
    if (epi == I8_NONE) PK_I8(I8_NONE);
    else if (epi == I8_GELU) PK_I8(I8_GELU);
    else PK_I8(I8_RESID);
#undef PK_I8
    PK_LAUNCH_CHECK("int8_gemm_kernel");
  }
  if (g.splits > 1) {
    const int64_t total = (int64_t)M * N;
    const bool vec = N % 8 == 0 && aligned16(g.partial) && aligned16(scale) && aligned16(C) &&
                     (epi != I8_RESID || aligned16(R));
    if (vec) {
      constexpr int T = PK_I8_REDUCE_THREADS;
      const int blocks = (int)std::min<int64_t>((total / 8 + T - 1) / T, 4096);
      if (epi == I8_NONE) int8_reduce8_kernel<I8_NONE><<<blocks, T, 0, st>>>(g);
      else if (epi == I8_GELU) int8_reduce8_kernel<I8_GELU><<<blocks, T, 0, st>>>(g);
      else int8_reduce8_kernel<I8_RESID><<<blocks, T, 0, st>>>(g);
    } else {
      const int blocks = (int)std::min<int64_t>((total + 255) / 256, 4096);
      if (epi == I8_NONE) int8_reduce_kernel<I8_NONE><<<blocks, 256, 0, st>>>(g);
      else if (epi == I8_GELU) int8_reduce_kernel<I8_GELU><<<blocks, 256, 0, st>>>(g);
      else int8_reduce_kernel<I8_RESID><<<blocks, 256, 0, st>>>(g);
    }
    PK_LAUNCH_CHECK("int8_reduce_kernel");
  }
  return PK_OK;
}

// ---- the no-allocation variant of launch_matmul_int8 -------------------------
// Split-K partials go to this file-scope device array instead of library or
// caller memory.  Every GPU the library runs on holds its own copy (16 MiB)
// until the process ends.  In host code `scratch` names a host-side stand-in,
// not device memory: its device address is looked up per device with
// hipGetSymbolAddress once (int8_scratch_setup) and only that address is
// passed to kernels.
constexpr size_t kInt8ScratchBytes = size_t(16) << 20;
static __device__ __align__(256) float scratch[kInt8ScratchBytes / sizeof(float)];

namespace {
constexpr int kScratchDevices = 64;
std::mutex g_scratch_mu;
void *g_scratch_ptr[kScratchDevices] = {};
}  // namespace

// Device address of the current device's `scratch` (looked up on the first
// call per device; later calls only read the table).
int int8_scratch_setup(void **out) {
  int dev = 0;
  PK_HIP(hipGetDevice(&dev));
  if (dev < 0 || dev >= kScratchDevices) {
    set_error("device ordinal %d out of range", dev);
    return PK_ERR_UNSUPPORTED;
  }
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void *p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) return hip_fail(e != hipSuccess ? e : hipErrorInvalidSymbol, "hipGetSymbolAddress(scratch)");
    g_scratch_ptr[dev] = p;
  }
  if (out) *out = g_scratch_ptr[dev];
  return PK_OK;
}

}  // namespace pk

using namespace pk;

extern "C" {

int launch_matmul_int8_noalloc(const uint16_t *A, const int8_t *Wq, const float *scale, uint16_t *C, int M, int N,
                               int K, void *stream) {
  PK_CHECK_ARG(A && Wq && scale && C, "launch_matmul_int8_noalloc: null tensor pointer");
  PK_CHECK_ARG(M >= 0 && N >= 0 && K > 0, "launch_matmul_int8_noalloc: invalid shape M=%d N=%d K=%d", M, N, K);
  if (M == 0 || N == 0) return PK_OK;
  const size_t need = int8_workspace_bytes(M, N, K);
  if (need > kInt8ScratchBytes) {
    set_error("launch_matmul_int8_noalloc: M=%d N=%d K=%d needs %zu bytes of split-K scratch, more than the %zu "
              "of the static buffer; use launch_matmul_int8 or pk_matmul_int8_ex with a workspace",
              M, N, K, need, kInt8ScratchBytes);
    return PK_ERR_WORKSPACE;
  }
  void *ws = nullptr;
  int rc = int8_scratch_setup(&ws);
  if (rc) return rc;
  // A caller workspace (the scratch) is never grown or replaced: int8_run
  // allocates nothing when it is given one.
  return int8_run(I8_NONE, A, Wq, scale, C, nullptr, M, N, K, nullptr, ws, kInt8ScratchBytes,
                  (hipStream_t)stream);
}

int launch_matmul_int8(const uint16_t *A, const int8_t *Wq, const float *scale, uint16_t *C,
                       int M, int N, int K, void *stream) {
  PK_CHECK_ARG(A && Wq && scale && C, "launch_matmul_int8: null tensor pointer");
  PK_CHECK_ARG(M >= 0 && N >= 0 && K > 0, "launch_matmul_int8: invalid shape M=%d N=%d K=%d", M, N, K);
  if (M == 0 || N == 0) return PK_OK;
  return int8_run(I8_NONE, A, Wq, scale, C, nullptr, M, N, K, nullptr, nullptr, 0, (hipStream_t)stream);
}

int pk_int8_default_config(int M, int N, int K, pk_config *out) {
  PK_CHECK_ARG(out && M > 0 && N > 0 && K > 0, "pk_int8_default_config: invalid argument");
  if (!int8_default(M, N, K, out)) {
    set_error("pk_int8_default_config: M=%d N=%d K=%d takes the generic kernel", M, N, K);
    return PK_ERR_UNSUPPORTED;
  }
  return PK_OK;
}

int pk_matmul_int8_ex(int epi, const uint16_t *A, const int8_t *Wq, const float *scale, uint16_t *C,
                      const uint16_t *R, int M, int N, int K, const pk_config *cfg,
                      void *workspace, size_t workspace_bytes, void *stream) {
  PK_CHECK_ARG(epi >= I8_NONE && epi <= I8_RESID, "pk_matmul_int8_ex: epilogue %d not in 0..2", epi);
  PK_CHECK_ARG(A && Wq && scale && C && (epi != I8_RESID || R), "pk_matmul_int8_ex: null tensor pointer");
  PK_CHECK_ARG(M >= 0 && N >= 0 && K > 0, "pk_matmul_int8_ex: invalid shape M=%d N=%d K=%d", M, N, K);
  if (M == 0 || N == 0) return PK_OK;
  return int8_run(epi, A, Wq, scale, C, R, M, N, K, cfg, workspace, workspace_bytes, (hipStream_t)stream);
}

size_t pk_decode_mlp_int8_workspace_size(int M, int d, int F) {
  if (M <= 0 || d <= 0 || F <= 0) return 0;  // no launch takes a workspace
  auto up = [](size_t v) { return (v + 255) & ~size_t(255); };
  const size_t p = std::max(int8_workspace_bytes(M, F, d), int8_workspace_bytes(M, d, F));
  return up((size_t)M * F * 2) + up(p);
}

int launch_decode_mlp_int8(const uint16_t *x, const int8_t *W1q, const float *s1,
                           const int8_t *W2q, const float *s2, uint16_t *out, int M, int d, int F,
                           void *workspace, size_t workspace_bytes, void *stream) {
  PK_CHECK_ARG(x && W1q && s1 && W2q && s2 && out, "launch_decode_mlp_int8: null tensor pointer");
  PK_CHECK_ARG(M >= 0 && d > 0 && F > 0, "launch_decode_mlp_int8: invalid shape");
  if (M == 0) return PK_OK;
  const size_t need = pk_decode_mlp_int8_workspace_size(M, d, F);
  if (!workspace || workspace_bytes < need) {
    set_error("launch_decode_mlp_int8: workspace of %zu bytes required, got %zu", need,
              workspace_bytes);
    return PK_ERR_WORKSPACE;
  }
  hipStream_t st = (hipStream_t)stream;
  const size_t hbytes = ((size_t)M * F * 2 + 255) & ~size_t(255);
  uint16_t *h = static_cast<uint16_t *>(workspace);
  void *part = static_cast<char *>(workspace) + hbytes;
  const size_t part_bytes = workspace_bytes - hbytes;
  int rc = int8_run(I8_GELU, x, W1q, s1, h, nullptr, M, F, d, nullptr, part, part_bytes, st);
  if (rc) return rc;
  return int8_run(I8_RESID, h, W2q, s2, out, x, M, d, F, nullptr, part, part_bytes, st);
}

}  // extern "C"
