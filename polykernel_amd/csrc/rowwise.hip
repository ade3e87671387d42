// rowwise.hip -- HBM-bound row kernels for gfx950: RMSNorm, residual+RMSNorm,
// softmax, masked softmax, GELU, KV append, int8 per-channel quantisation.
//
// One row per wave (short rows) or per 256-thread block (long rows), the row
// held in registers so every input byte is read from HBM exactly once; 16-byte
// vector loads/stores; wave64 shuffle reductions, then one LDS exchange across
// the block's 4 waves.
#include "pk_common.hpp"

namespace pk {

namespace {

constexpr int kBlock = 256;

struct alignas(16) U4 {
  uint32_t x, y, z, w;
};

__device__ __forceinline__ U4 ld16(const void *p) { return *reinterpret_cast<const U4 *>(p); }
__device__ __forceinline__ void st16(void *p, U4 v) { *reinterpret_cast<U4 *>(p) = v; }
// 16-byte load of data read exactly once (the rows of x, r, logits, mask):
// non-temporal, so the stream does not allocate in the caches.  Measured on
// MI355X: residual+RMSNorm [16384, 8192] 143 -> 123 us, masked softmax
// 197 -> 169 us (the same hint on the stores made both slower).
typedef uint32_t nt_u32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ U4 ld16_once(const void *p) {
  return __builtin_bit_cast(U4, __builtin_nontemporal_load(reinterpret_cast<const nt_u32x4 *>(p)));
}

__device__ __forceinline__ void unpack8(U4 v, float (&f)[8]) {
  f[0] = lo_bf(v.x), f[1] = hi_bf(v.x), f[2] = lo_bf(v.y), f[3] = hi_bf(v.y);
  f[4] = lo_bf(v.z), f[5] = hi_bf(v.z), f[6] = lo_bf(v.w), f[7] = hi_bf(v.w);
}

__device__ __forceinline__ U4 pack8(const float (&f)[8]) {
  return U4{pack_bf(f[0], f[1]), pack_bf(f[2], f[3]), pack_bf(f[4], f[5]), pack_bf(f[6], f[7])};
}

// Sum over the block's waves (NW == 1: just the wave sum).
template <int NW>
__device__ __forceinline__ float group_sum(float v, float *red) {
  v = wave_sum(v);
  if constexpr (NW == 1) {
    return v;
  } else {
    const int w = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[w] = v;
    __syncthreads();
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < NW; ++i) s += red[i];
    return s;
  }
}

template <int NW>
__device__ __forceinline__ float group_max(float v, float *red) {
  v = wave_max(v);
  if constexpr (NW == 1) {
    return v;
  } else {
    const int w = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[w] = v;
    __syncthreads();
    float s = red[0];
#pragma unroll
    for (int i = 1; i < NW; ++i) s = fmaxf(s, red[i]);
    return s;
  }
}

__global__ __launch_bounds__(kBlock) void div_check_kernel(const float *__restrict__ ds, int n,
                                                           unsigned long long *__restrict__ bad) {
  const int64_t t = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  if (t >= (int64_t)n * 65536) return;
  const float d = ds[t >> 16];
  const float x = bf2f((uint32_t)(t & 0xFFFF));
  if (!div_row_ok(d) || !div_elem_ok(x)) return;
  const float want = x / d, got = div_fast(x, d, 1.0f / d);
  if (__float_as_uint(want) != __float_as_uint(got)) atomicAdd(bad, 1ull);
}

// ---------------------------------------------------------------------------
// RMSNorm / residual + RMSNorm (vector path: cols % 8 == 0, 16-byte aligned).
// NW waves cooperate on one row (NW == 1: each wave owns a row, 4 rows per
// block).  Each lane keeps VPT 8-element vectors of the row in registers.
// Arithmetic per kernels/cpu/cpu_reference.cpp:16-44: ss = sum x^2 (fp32),
// rms = sqrt(ss * (1/cols) + eps), y = bf16((x / rms) [* w]).  With a residual
// the normalised value is s = bf16(x + r) (tests/golden/golden.py:108-112).
// ---------------------------------------------------------------------------
template <int NW, int VPT, bool RESID>
__global__ __launch_bounds__(kBlock) void rmsnorm_vec_kernel(const uint16_t *__restrict__ x,
                                                             const uint16_t *__restrict__ r,
                                                             const uint16_t *__restrict__ w,
                                                             uint16_t *__restrict__ y, int rows,
                                                             int cols, float inv_cols, float eps) {
#pragma clang fp contract(off)
  __shared__ float red[NW];
  constexpr int kRowsPerBlock = (NW == 1) ? (kBlock / 64) : 1;
  constexpr int kLanes = NW * 64;
  const int row = (NW == 1) ? (blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6)) : blockIdx.x;
  const int lane = (NW == 1) ? (threadIdx.x & 63) : threadIdx.x;
  if (row >= rows) return;  // uniform per row-group (NW == 1: per wave)
  const int nvec = cols >> 3;
  const size_t base = (size_t)row * cols;

  float v[VPT][8];
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    const int c = lane + i * kLanes;
    if (c < nvec) {
      unpack8(ld16_once(x + base + (size_t)c * 8), v[i]);
      if constexpr (RESID) {
        float rv[8];
        unpack8(ld16_once(r + base + (size_t)c * 8), rv);
#pragma unroll
        for (int e = 0; e < 8; ++e) v[i][e] = bf2f(f2bf(v[i][e] + rv[e]));
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) ss += v[i][e] * v[i][e];
    }
  }
  ss = group_sum<NW>(ss, red);
  const float rms = sqrtf(ss * inv_cols + eps);
  // x / rms with the fast exact division when every element of the wave allows it
  bool ok = div_row_ok(rms);
#pragma unroll
  for (int i = 0; i < VPT; ++i)
    if (lane + i * kLanes < nvec)
#pragma unroll
      for (int e = 0; e < 8; ++e) ok &= div_elem_ok(v[i][e]);
  const bool fast = __all(ok);
  const float rinv = 1.0f / rms;
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    const int c = lane + i * kLanes;
    if (c < nvec) {
      float o[8];
      if (fast) {
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = div_fast(v[i][e], rms, rinv);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = v[i][e] / rms;
      }
      if (w) {
        float g[8];
        unpack8(ld16(w + (size_t)c * 8), g);
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] *= g[e];
      }
      st16(y + base + (size_t)c * 8, pack8(o));
    }
  }
}

// Generic path (any cols / alignment): one block per row, two passes over the
// row (the second from cache).
template <bool RESID>
__global__ __launch_bounds__(kBlock) void rmsnorm_generic_kernel(
    const uint16_t *__restrict__ x, const uint16_t *__restrict__ r, const uint16_t *__restrict__ w,
    uint16_t *__restrict__ y, int rows, int cols, float inv_cols, float eps) {
#pragma clang fp contract(off)
  __shared__ float red[kBlock / 64];
  const int row = blockIdx.x;
  const size_t base = (size_t)row * cols;
  float ss = 0.f;
  for (int c = threadIdx.x; c < cols; c += kBlock) {
    float s = bf2f(x[base + c]);
    if constexpr (RESID) s = bf2f(f2bf(s + bf2f(r[base + c])));
    ss += s * s;
  }
  ss = group_sum<kBlock / 64>(ss, red);
  const float rms = sqrtf(ss * inv_cols + eps);
  for (int c = threadIdx.x; c < cols; c += kBlock) {
    float s = bf2f(x[base + c]);
    if constexpr (RESID) s = bf2f(f2bf(s + bf2f(r[base + c])));
    float o = s / rms;
    if (w) o *= bf2f(w[c]);
    y[base + c] = (uint16_t)f2bf(o);
  }
}

template <bool RESID>
int rmsnorm_dispatch(const uint16_t *x, const uint16_t *r, const uint16_t *w, uint16_t *y,
                     int rows, int cols, float eps, hipStream_t st, const char *name) {
  PK_CHECK_ARG(x && y && (!RESID || r), "%s: null tensor pointer", name);
  PK_CHECK_ARG(rows >= 0 && cols > 0, "%s: invalid shape rows=%d cols=%d", name, rows, cols);
  if (rows == 0) return PK_OK;
  const float inv_cols = 1.0f / (float)cols;
  const bool vec = (cols % 8 == 0) && aligned16(x) && aligned16(y) && (!RESID || aligned16(r)) &&
                   (!w || aligned16(w));
  const int nvec = cols / 8;
  if (vec && nvec <= 64 * 8) {
    // one wave per row, 4 rows per block
    const dim3 grid((rows + 3) / 4);
#define PK_RMS_W(VPT)                                                                       \
  rmsnorm_vec_kernel<1, VPT, RESID><<<grid, kBlock, 0, st>>>(x, r, w, y, rows, cols, inv_cols, eps)
    if (nvec <= 64) PK_RMS_W(1);
    else if (nvec <= 128) PK_RMS_W(2);
    else if (nvec <= 256) PK_RMS_W(4);
    else PK_RMS_W(8);
#undef PK_RMS_W
  } else if (vec && nvec <= 256 * 8) {
    const dim3 grid(rows);
#define PK_RMS_B(VPT)                                                                       \
  rmsnorm_vec_kernel<4, VPT, RESID><<<grid, kBlock, 0, st>>>(x, r, w, y, rows, cols, inv_cols, eps)
    if (nvec <= 256 * 4) PK_RMS_B(4);
    else PK_RMS_B(8);
#undef PK_RMS_B
  } else {
    rmsnorm_generic_kernel<RESID><<<rows, kBlock, 0, st>>>(x, r, w, y, rows, cols, inv_cols, eps);
  }
  PK_LAUNCH_CHECK(name);
  return PK_OK;
}

// ---------------------------------------------------------------------------
// Softmax over the last axis.  MODE 0: bf16 input (kernels/cpu/cpu_reference.cpp:107-128);
// MODE 1: fp32 logits + bf16 additive mask, z = bf16(bf16(x) + mask)
// (tests/golden/golden.py:115-117).  m = max z, e = exp(z - m), y = bf16(e * (1/sum e)).
// ---------------------------------------------------------------------------
template <int MODE>
__device__ __forceinline__ void load_z8(const void *in, const uint16_t *mask, size_t off,
                                        float (&z)[8]) {
  if constexpr (MODE == 0) {
    unpack8(ld16_once(static_cast<const uint16_t *>(in) + off), z);
  } else {
    const float *xf = static_cast<const float *>(in) + off;
    const U4 a = ld16_once(xf), b = ld16_once(xf + 4);
    float m[8];
    unpack8(ld16_once(mask + off), m);
    const uint32_t raw[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
    for (int e = 0; e < 8; ++e) z[e] = bf2f(f2bf(bf2f(f2bf(__uint_as_float(raw[e]))) + m[e]));
  }
}

template <int MODE>
__device__ __forceinline__ float load_z1(const void *in, const uint16_t *mask, size_t off) {
  if constexpr (MODE == 0) {
    return bf2f(static_cast<const uint16_t *>(in)[off]);
  } else {
    const float xb = bf2f(f2bf(static_cast<const float *>(in)[off]));
    return bf2f(f2bf(xb + bf2f(mask[off])));
  }
}

template <int NW, int VPT, int MODE>
__global__ __launch_bounds__(kBlock) void softmax_vec_kernel(const void *__restrict__ in,
                                                             const uint16_t *__restrict__ mask,
                                                             uint16_t *__restrict__ y, int rows,
                                                             int cols) {
#pragma clang fp contract(off)
  __shared__ float red[NW];
  constexpr int kRowsPerBlock = (NW == 1) ? (kBlock / 64) : 1;
  constexpr int kLanes = NW * 64;
  const int row = (NW == 1) ? (blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6)) : blockIdx.x;
  const int lane = (NW == 1) ? (threadIdx.x & 63) : threadIdx.x;
  if (row >= rows) return;
  const int nvec = cols >> 3;
  const size_t base = (size_t)row * cols;

  float z[VPT][8];
  float m = -INFINITY;
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    const int c = lane + i * kLanes;
    if (c < nvec) {
      load_z8<MODE>(in, mask, base + (size_t)c * 8, z[i]);
#pragma unroll
      for (int e = 0; e < 8; ++e) m = fmaxf(m, z[i][e]);
    }
  }
  m = group_max<NW>(m, red);
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    const int c = lane + i * kLanes;
    if (c < nvec) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        z[i][e] = expf(z[i][e] - m);
        s += z[i][e];
      }
    }
  }
  s = group_sum<NW>(s, red);
  const float inv = 1.0f / s;
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    const int c = lane + i * kLanes;
    if (c < nvec) {
      float o[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = z[i][e] * inv;
      st16(y + base + (size_t)c * 8, pack8(o));
    }
  }
}

template <int MODE>
__global__ __launch_bounds__(kBlock) void softmax_generic_kernel(const void *__restrict__ in,
                                                                 const uint16_t *__restrict__ mask,
                                                                 uint16_t *__restrict__ y,
                                                                 int rows, int cols) {
#pragma clang fp contract(off)
  __shared__ float red[kBlock / 64];
  const int row = blockIdx.x;
  const size_t base = (size_t)row * cols;
  float m = -INFINITY;
  for (int c = threadIdx.x; c < cols; c += kBlock) m = fmaxf(m, load_z1<MODE>(in, mask, base + c));
  m = group_max<kBlock / 64>(m, red);
  float s = 0.f;
  for (int c = threadIdx.x; c < cols; c += kBlock) s += expf(load_z1<MODE>(in, mask, base + c) - m);
  s = group_sum<kBlock / 64>(s, red);
  const float inv = 1.0f / s;
  for (int c = threadIdx.x; c < cols; c += kBlock)
    y[base + c] = (uint16_t)f2bf(expf(load_z1<MODE>(in, mask, base + c) - m) * inv);
}

template <int MODE>
int softmax_dispatch(const void *in, const uint16_t *mask, uint16_t *y, int rows, int cols,
                     hipStream_t st, const char *name) {
  PK_CHECK_ARG(in && y && (MODE == 0 || mask), "%s: null tensor pointer", name);
  PK_CHECK_ARG(rows >= 0 && cols > 0, "%s: invalid shape rows=%d cols=%d", name, rows, cols);
  if (rows == 0) return PK_OK;
  const bool vec = (cols % 8 == 0) && aligned16(in) && aligned16(y) && (MODE == 0 || aligned16(mask));
  const int nvec = cols / 8;
  if (vec && nvec <= 64 * 4) {
    const dim3 grid((rows + 3) / 4);
#define PK_SM_W(VPT) softmax_vec_kernel<1, VPT, MODE><<<grid, kBlock, 0, st>>>(in, mask, y, rows, cols)
    if (nvec <= 64) PK_SM_W(1);
    else if (nvec <= 128) PK_SM_W(2);
    else PK_SM_W(4);
#undef PK_SM_W
  } else if (vec && nvec <= 256 * 8) {
    const dim3 grid(rows);
#define PK_SM_B(VPT) softmax_vec_kernel<4, VPT, MODE><<<grid, kBlock, 0, st>>>(in, mask, y, rows, cols)
    if (nvec <= 256 * 2) PK_SM_B(2);
    else if (nvec <= 256 * 4) PK_SM_B(4);
    else PK_SM_B(8);
#undef PK_SM_B
  } else {
    softmax_generic_kernel<MODE><<<rows, kBlock, 0, st>>>(in, mask, y, rows, cols);
  }
  PK_LAUNCH_CHECK(name);
  return PK_OK;
}

// ---------------------------------------------------------------------------
// GELU: out = gelu_bits(in)  (kernels/cpu/cpu_reference.cpp:46-55, exact).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kBlock) void gelu_kernel(const uint16_t *__restrict__ in,
                                                      uint16_t *__restrict__ out, int64_t n,
                                                      const uint16_t *__restrict__ tab) {
  const int64_t nvec = n >> 3;
  const int64_t stride = (int64_t)gridDim.x * kBlock;
  for (int64_t v = (int64_t)blockIdx.x * kBlock + threadIdx.x; v < nvec; v += stride) {
    U4 a = ld16(in + v * 8);
    uint32_t w[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
    for (int j = 0; j < 4; ++j)
      w[j] = gelu_bits(w[j] & 0xFFFFu, tab) | (gelu_bits(w[j] >> 16, tab) << 16);
    st16(out + v * 8, U4{w[0], w[1], w[2], w[3]});
  }
  for (int64_t i = nvec * 8 + (int64_t)blockIdx.x * kBlock + threadIdx.x; i < n; i += stride)
    out[i] = (uint16_t)gelu_bits(in[i], tab);
}

__global__ __launch_bounds__(kBlock) void gelu_scalar_kernel(const uint16_t *__restrict__ in,
                                                             uint16_t *__restrict__ out, int64_t n,
                                                             const uint16_t *__restrict__ tab) {
  const int64_t stride = (int64_t)gridDim.x * kBlock;
  for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < n; i += stride)
    out[i] = (uint16_t)gelu_bits(in[i], tab);
}

// ---------------------------------------------------------------------------
// KV-cache append (kernels/cpu/attention.cpp:63-92): a verbatim bf16 copy.
// Rows of D elements; 16-byte vectors when D % 8 == 0.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kBlock) void kv_concat_kernel(const uint16_t *__restrict__ cache,
                                                           const uint16_t *__restrict__ neu,
                                                           uint16_t *__restrict__ out, int64_t BH,
                                                           int64_t Sc, int64_t Sn, int64_t D,
                                                           int vec) {
  const int64_t S = Sc + Sn;
  const int64_t per = vec ? D / 8 : D;  // units per row
  const int64_t total = BH * S * per;
  const int64_t stride = (int64_t)gridDim.x * kBlock;
  for (int64_t t = (int64_t)blockIdx.x * kBlock + threadIdx.x; t < total; t += stride) {
    const int64_t u = t % per, rs = t / per, s = rs % S, bh = rs / S;
    const uint16_t *src =
        (s < Sc) ? cache + (bh * Sc + s) * D : neu + (bh * Sn + (s - Sc)) * D;
    uint16_t *dst = out + (bh * S + s) * D;
    if (vec) st16(dst + u * 8, ld16(src + u * 8));
    else dst[u] = src[u];
  }
}

// ---------------------------------------------------------------------------
// int8 per-output-channel quantisation (tests/golden/quant_golden.py:71-83).
// Pass 1: amax[n] = max_k |W[k,n]| as float bits (non-negative floats order
// like their bit patterns, so atomicMax on uint32 is exact and order-free).
// Pass 2: scale[n] = amax > 0 ? amax / 127 : 1.  Pass 3: wq = clip(rint(w / scale)).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kBlock) void fill_u32_kernel(uint32_t *p, int n, uint32_t v) {
  const int i = blockIdx.x * kBlock + threadIdx.x;
  if (i < n) p[i] = v;
}

constexpr int kQuantRows = 128;

__global__ __launch_bounds__(kBlock) void quant_amax_kernel(const uint16_t *__restrict__ W,
                                                            uint32_t *__restrict__ amax_bits, int K,
                                                            int N) {
  const int n = blockIdx.x * kBlock + threadIdx.x;
  if (n >= N) return;
  const int k0 = blockIdx.y * kQuantRows;
  const int k1 = min(K, k0 + kQuantRows);
  uint32_t m = 0;
  for (int k = k0; k < k1; ++k) m = max(m, (uint32_t)W[(size_t)k * N + n] & 0x7FFFu);
  // bf16 magnitude bits -> fp32 bits (exact upcast); max of non-negative floats.
  atomicMax(amax_bits + n, m << 16);
}

__global__ __launch_bounds__(kBlock) void quant_scale_kernel(const uint32_t *__restrict__ amax_bits,
                                                             float *__restrict__ scale, int N) {
  const int n = blockIdx.x * kBlock + threadIdx.x;
  if (n >= N) return;
  const float amax = __uint_as_float(amax_bits[n]);
  scale[n] = (amax > 0.0f) ? amax / 127.0f : 1.0f;
}

__global__ __launch_bounds__(kBlock) void quant_apply_kernel(const uint16_t *__restrict__ W,
                                                             const float *__restrict__ scale,
                                                             int8_t *__restrict__ Wq, int K, int N) {
  const int64_t total = (int64_t)K * N;
  const int64_t stride = (int64_t)gridDim.x * kBlock;
  for (int64_t t = (int64_t)blockIdx.x * kBlock + threadIdx.x; t < total; t += stride) {
    const int n = (int)(t % N);
    float q = rintf(bf2f(W[t]) / scale[n]);
    q = fminf(fmaxf(q, -127.0f), 127.0f);
    Wq[t] = (int8_t)(int)q;
  }
}

int grid_for(int64_t work, int per_thread = 1) {
  int64_t b = (work / per_thread + kBlock - 1) / kBlock;
  return (int)std::min<int64_t>(std::max<int64_t>(b, 1), 256 * 64);
}

}  // namespace

// exported to other translation units (mlp block)
int rmsnorm_launch(const uint16_t *x, const uint16_t *w, uint16_t *y, int rows, int cols,
                   float eps, hipStream_t st) {
  return rmsnorm_dispatch<false>(x, nullptr, w, y, rows, cols, eps, st, "rmsnorm");
}

int gelu_launch(const uint16_t *in, uint16_t *out, int64_t n, hipStream_t st) {
  const uint16_t *tab = nullptr;
  int rc = gelu_table(&tab);
  if (rc) return rc;
  if (n == 0) return PK_OK;
  if (aligned16(in) && aligned16(out)) gelu_kernel<<<grid_for(n, 8), kBlock, 0, st>>>(in, out, n, tab);
  else gelu_scalar_kernel<<<grid_for(n), kBlock, 0, st>>>(in, out, n, tab);
  PK_LAUNCH_CHECK("gelu");
  return PK_OK;
}

// The kernels the row-wise dispatchers above run for 16-byte aligned
// operands, as configs: block_m = rows per workgroup (4: one wave per row;
// 1: four waves per row), block_n = cols, num_warps = 4, vector_width = bf16
// per load (8, or 1 for the generic kernel), unroll = 16-byte vectors per
// lane, one pass over a register-resident row (block_k 0, stages 1).
bool rmsnorm_config(int rows, int cols, pk_config *out) {
  if (rows <= 0 || cols <= 0) return false;
  const int nvec = cols / 8;
  if (cols % 8 == 0 && nvec <= 64 * 8) {
    const int vpt = nvec <= 64 ? 1 : nvec <= 128 ? 2 : nvec <= 256 ? 4 : 8;
    *out = pk_config{4, cols, 0, kBlock / 64, 8, vpt, 1};
  } else if (cols % 8 == 0 && nvec <= 256 * 8) {
    *out = pk_config{1, cols, 0, kBlock / 64, 8, nvec <= 256 * 4 ? 4 : 8, 1};
  } else {
    *out = pk_config{1, cols, 0, kBlock / 64, 1, 1, 1};
  }
  return true;
}

bool softmax_config(int rows, int cols, pk_config *out) {
  if (rows <= 0 || cols <= 0) return false;
  const int nvec = cols / 8;
  if (cols % 8 == 0 && nvec <= 64 * 4) {
    *out = pk_config{4, cols, 0, kBlock / 64, 8, nvec <= 64 ? 1 : nvec <= 128 ? 2 : 4, 1};
  } else if (cols % 8 == 0 && nvec <= 256 * 8) {
    *out = pk_config{1, cols, 0, kBlock / 64, 8, nvec <= 256 * 2 ? 2 : nvec <= 256 * 4 ? 4 : 8, 1};
  } else {
    *out = pk_config{1, cols, 0, kBlock / 64, 1, 1, 1};
  }
  return true;
}

}  // namespace pk

using namespace pk;

extern "C" {

int launch_rmsnorm(const uint16_t *input, const uint16_t *weight, uint16_t *output, int rows,
                   int cols, float eps, void *stream) {
  return rmsnorm_dispatch<false>(input, nullptr, weight, output, rows, cols, eps,
                                 (hipStream_t)stream, "launch_rmsnorm");
}

int launch_fused_residual_rmsnorm(const uint16_t *x, const uint16_t *r, const uint16_t *gamma,
                                  uint16_t *out, int rows, int cols, float eps, void *stream) {
  return rmsnorm_dispatch<true>(x, r, gamma, out, rows, cols, eps, (hipStream_t)stream,
                                "launch_fused_residual_rmsnorm");
}

int launch_softmax(const uint16_t *input, uint16_t *output, int rows, int cols, void *stream) {
  return softmax_dispatch<0>(input, nullptr, output, rows, cols, (hipStream_t)stream,
                             "launch_softmax");
}

int launch_fused_softmax_mask(const float *logits, const uint16_t *mask, uint16_t *out, int rows,
                              int cols, void *stream) {
  return softmax_dispatch<1>(logits, mask, out, rows, cols, (hipStream_t)stream,
                             "launch_fused_softmax_mask");
}

int launch_gelu(const uint16_t *input, uint16_t *output, int n, void *stream) {
  PK_CHECK_ARG(input && output && n >= 0, "launch_gelu: invalid arguments");
  return gelu_launch(input, output, n, (hipStream_t)stream);
}

int launch_kv_cache_update(const uint16_t *cache, const uint16_t *new_rows, uint16_t *out, int B,
                           int H, int S_cache, int S_new, int D, void *stream) {
  PK_CHECK_ARG(out && (S_cache == 0 || cache) && (S_new == 0 || new_rows),
               "launch_kv_cache_update: null tensor pointer");
  PK_CHECK_ARG(B >= 0 && H >= 0 && S_cache >= 0 && S_new >= 0 && D > 0,
               "launch_kv_cache_update: invalid shape");
  const int64_t BH = (int64_t)B * H;
  const int64_t S = (int64_t)S_cache + S_new;
  if (BH * S == 0) return PK_OK;
  const int vec = (D % 8 == 0) && aligned16(out) && (S_cache == 0 || aligned16(cache)) &&
                  (S_new == 0 || aligned16(new_rows));
  const int64_t units = BH * S * (vec ? D / 8 : D);
  kv_concat_kernel<<<grid_for(units), kBlock, 0, (hipStream_t)stream>>>(cache, new_rows, out, BH,
                                                                         S_cache, S_new, D, vec);
  PK_LAUNCH_CHECK("launch_kv_cache_update");
  return PK_OK;
}

int launch_quantize_int8_per_channel(const uint16_t *W, int8_t *Wq, float *scale, int K, int N,
                                     void *stream) {
  PK_CHECK_ARG(W && Wq && scale, "launch_quantize_int8_per_channel: null tensor pointer");
  PK_CHECK_ARG(K > 0 && N > 0, "launch_quantize_int8_per_channel: invalid shape K=%d N=%d", K, N);
  hipStream_t st = (hipStream_t)stream;
  // The per-channel amax bits are staged in `scale` itself (same size, fp32).
  uint32_t *amax_bits = reinterpret_cast<uint32_t *>(scale);
  fill_u32_kernel<<<(N + kBlock - 1) / kBlock, kBlock, 0, st>>>(amax_bits, N, 0u);
  dim3 g1((N + kBlock - 1) / kBlock, (K + kQuantRows - 1) / kQuantRows);
  quant_amax_kernel<<<g1, kBlock, 0, st>>>(W, amax_bits, K, N);
  quant_scale_kernel<<<(N + kBlock - 1) / kBlock, kBlock, 0, st>>>(amax_bits, scale, N);
  quant_apply_kernel<<<grid_for((int64_t)K * N), kBlock, 0, st>>>(W, scale, Wq, K, N);
  PK_LAUNCH_CHECK("launch_quantize_int8_per_channel");
  return PK_OK;
}

int pk_check_row_division(const float *divisors, int n, unsigned long long *mismatches) {
  PK_CHECK_ARG(divisors && mismatches && n >= 0 && n <= 32768, "pk_check_row_division: invalid argument");
  *mismatches = 0;
  if (n == 0) return PK_OK;
  float *dd = nullptr;
  unsigned long long *bad = nullptr;
  PK_HIP(hipMalloc(&dd, (size_t)n * sizeof(float)));
  hipError_t e = hipMalloc(&bad, sizeof *bad);
  if (e == hipSuccess) e = hipMemcpy(dd, divisors, (size_t)n * sizeof(float), hipMemcpyHostToDevice);
  if (e == hipSuccess) e = hipMemset(bad, 0, sizeof *bad);
  if (e == hipSuccess) {
    div_check_kernel<<<(int)(((int64_t)n * 65536 + kBlock - 1) / kBlock), kBlock>>>(dd, n, bad);
    e = hipGetLastError();
  }
  if (e == hipSuccess) e = hipMemcpy(mismatches, bad, sizeof *bad, hipMemcpyDeviceToHost);
  (void)hipFree(dd);
  if (bad) (void)hipFree(bad);
  return e == hipSuccess ? PK_OK : hip_fail(e, "pk_check_row_division");
}

}  // extern "C"
