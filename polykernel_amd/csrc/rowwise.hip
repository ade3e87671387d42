// rowwise.hip -- HBM-bound row kernels for gfx950: RMSNorm, residual+RMSNorm,
// softmax, masked softmax (bodies in rowwise_kernels.hpp), GELU, KV append,
// int8 per-channel quantisation, and their launchers.
#include "rowwise_kernels.hpp"

namespace pk {

namespace {

using namespace row;

__global__ __launch_bounds__(kBlock) void div_check_kernel(const float *__restrict__ ds, int n,
                                                           unsigned long long *__restrict__ bad) {
  const int64_t t = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  if (t >= (int64_t)n * 65536) return;
  const float d = ds[t >> 16];
  const uint32_t code = (uint32_t)(t & 0xFFFF);
  const float x = bf2f(code);
  if ((t >> 16) == 0) {
    // once per numerator code: the packed magnitude test (DivSpan) accepts
    // exactly the codes with 2^-64 <= |x| < 2^64, whether the code is paired
    // with itself or with an in-range code (1.0) in its 32-bit word
    DivSpan self, mixed;
    div_span_add(self, code | (code << 16));
    div_span_add(mixed, code | (0x3F80u << 16));
    const bool want = div_elem_ok(x) && fabsf(x) < 0x1p64f;
    if (div_span_ok(self) != want || div_span_ok(mixed) != want) atomicAdd(bad, 1ull);
  }
  if (!div_row_ok(d) || !div_elem_ok(x)) return;
  const float want = x / d, got = div_fast(x, d, 1.0f / d);
  if (__float_as_uint(want) != __float_as_uint(got)) atomicAdd(bad, 1ull);
}

// The row kernels, as the library launches them (bodies in rowwise_kernels.hpp).
template <int NW, int VPT, bool RESID>
__global__ __launch_bounds__(kBlock) void rmsnorm_vec_kernel(RowArgs a) {
  rmsnorm_vec_body<NW, VPT, RESID>(a);
}

template <bool RESID>
__global__ __launch_bounds__(kBlock) void rmsnorm_generic_kernel(RowArgs a) {
  rmsnorm_generic_body<RESID>(a);
}

template <bool RESID>
int rmsnorm_dispatch(const uint16_t *x, const uint16_t *r, const uint16_t *w, uint16_t *y,
                     int rows, int cols, float eps, hipStream_t st, const char *name) {
  PK_CHECK_ARG(x && y && (!RESID || r), "%s: null tensor pointer", name);
  PK_CHECK_ARG(rows >= 0 && cols > 0, "%s: invalid shape rows=%d cols=%d", name, rows, cols);
  if (rows == 0) return PK_OK;
  const RowArgs a{x, RESID ? r : nullptr, w, y, rows, cols, 1.0f / (float)cols, eps};
  const bool vec = (cols % 8 == 0) && aligned16(x) && aligned16(y) && (!RESID || aligned16(r)) &&
                   (!w || aligned16(w));
  const int nvec = cols / 8;
  if (vec && nvec <= 64 * 8) {
    // one wave per row, 4 rows per block
    const dim3 grid(rows / 4 + (rows % 4 != 0));
#define PK_RMS_W(VPT) rmsnorm_vec_kernel<1, VPT, RESID><<<grid, kBlock, 0, st>>>(a)
    if (nvec <= 64) PK_RMS_W(1);
    else if (nvec <= 128) PK_RMS_W(2);
    else if (nvec <= 256) PK_RMS_W(4);
    else PK_RMS_W(8);
#undef PK_RMS_W
  } else if (vec && nvec <= 256 * 8) {
    const dim3 grid(rows);
#define PK_RMS_B(VPT) rmsnorm_vec_kernel<4, VPT, RESID><<<grid, kBlock, 0, st>>>(a)
    if (nvec <= 256 * 4) PK_RMS_B(4);
    else PK_RMS_B(8);
#undef PK_RMS_B
  } else {
    rmsnorm_generic_kernel<RESID><<<rows, kBlock, 0, st>>>(a);
  }
  PK_LAUNCH_CHECK(name);
  return PK_OK;
}

template <int NW, int VPT, int MODE>
__global__ __launch_bounds__(kBlock) void softmax_vec_kernel(RowArgs a) {
  softmax_vec_body<NW, VPT, MODE>(a);
}

template <int MODE>
__global__ __launch_bounds__(kBlock) void softmax_generic_kernel(RowArgs a) {
  softmax_generic_body<MODE>(a);
}

template <int MODE>
int softmax_dispatch(const void *in, const uint16_t *mask, uint16_t *y, int rows, int cols,
                     hipStream_t st, const char *name) {
  PK_CHECK_ARG(in && y && (MODE == 0 || mask), "%s: null tensor pointer", name);
  PK_CHECK_ARG(rows >= 0 && cols > 0, "%s: invalid shape rows=%d cols=%d", name, rows, cols);
  if (rows == 0) return PK_OK;
  const RowArgs a{in, MODE == 0 ? nullptr : mask, nullptr, y, rows, cols, 0.f, 0.f};
  const bool vec = (cols % 8 == 0) && aligned16(in) && aligned16(y) && (MODE == 0 || aligned16(mask));
  const int nvec = cols / 8;
  if (vec && nvec <= 64 * 4) {
    const dim3 grid(rows / 4 + (rows % 4 != 0));
#define PK_SM_W(VPT) softmax_vec_kernel<1, VPT, MODE><<<grid, kBlock, 0, st>>>(a)
    if (nvec <= 64) PK_SM_W(1);
    else if (nvec <= 128) PK_SM_W(2);
    else PK_SM_W(4);
#undef PK_SM_W
  } else if (vec && nvec <= 256 * 8) {
    const dim3 grid(rows);
#define PK_SM_B(VPT) softmax_vec_kernel<4, VPT, MODE><<<grid, kBlock, 0, st>>>(a)
    if (nvec <= 256 * 2) PK_SM_B(2);
    else if (nvec <= 256 * 4) PK_SM_B(4);
    else PK_SM_B(8);
#undef PK_SM_B
  } else {
    softmax_generic_kernel<MODE><<<rows, kBlock, 0, st>>>(a);
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
  uint32_t m = 0;
  // chunks of kQuantRows rows, strided by the grid's y extent (at most 65535)
  for (int64_t k0 = (int64_t)blockIdx.y * kQuantRows; k0 < K; k0 += (int64_t)gridDim.y * kQuantRows) {
    const int64_t k1 = min((int64_t)K, k0 + kQuantRows);
    for (int64_t k = k0; k < k1; ++k) m = max(m, (uint32_t)W[(size_t)k * N + n] & 0x7FFFu);
  }
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
  PK_CHECK_ARG(N <= INT32_MAX - kBlock, "launch_quantize_int8_per_channel: N=%d is within %d of INT32_MAX", N,
               kBlock);
  hipStream_t st = (hipStream_t)stream;
  // The per-channel amax bits are staged in `scale` itself (same size, fp32).
  uint32_t *amax_bits = reinterpret_cast<uint32_t *>(scale);
  fill_u32_kernel<<<(N + kBlock - 1) / kBlock, kBlock, 0, st>>>(amax_bits, N, 0u);
  dim3 g1((N + kBlock - 1) / kBlock, (unsigned)std::min<int64_t>(((int64_t)K + kQuantRows - 1) / kQuantRows, 65535));
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
