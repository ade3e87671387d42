// rowwise.hip -- HBM-bound row kernels for gfx950: RMSNorm, residual+RMSNorm,
// softmax, masked softmax (bodies in rowwise_kernels.hpp), GELU, KV append,
// int8 per-channel quantisation, and their launchers.
#include <algorithm>
#include <cstring>

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
// NW waves per row (NW == 1: one wave per row, 4 rows per 256-thread block;
// otherwise one row per NW * 64-thread block), VPT 16-byte vectors per lane.
template <int NW, int VPT, bool RESID>
__global__ __launch_bounds__(NW > 4 ? NW * 64 : kBlock) void rmsnorm_vec_kernel(RowArgs a) {
  rmsnorm_vec_body<NW, VPT, RESID>(a);
}

template <bool RESID>
__global__ __launch_bounds__(kBlock) void rmsnorm_generic_kernel(RowArgs a) {
  rmsnorm_generic_body<RESID>(a);
}

template <int NW, int VPT, int MODE>
__global__ __launch_bounds__(NW > 4 ? NW * 64 : kBlock) void softmax_vec_kernel(RowArgs a) {
  softmax_vec_body<NW, VPT, MODE>(a);
}

template <int MODE>
__global__ __launch_bounds__(kBlock) void softmax_generic_kernel(RowArgs a) {
  softmax_generic_body<MODE>(a);
}

// Rows of up to 131072 columns: 16 waves, the row as packed bf16 in registers.
template <bool RESID>
__global__ __launch_bounds__(kPackedLanes) void rmsnorm_packed_kernel(RowArgs a) {
  rmsnorm_packed_body<RESID>(a);
}

template <int MODE>
__global__ __launch_bounds__(kPackedLanes) void softmax_packed_kernel(RowArgs a) {
  softmax_packed_body<MODE>(a);
}

// ---- configurations ---------------------------------------------------------
// A row config: block_m = rows per workgroup (4: one wave per row; 1: one
// row per workgroup of num_warps waves, 4, 8 or 16), block_n = cols, num_warps,
// vector_width = bf16 per load (8; 1 for the generic kernel, any cols and
// alignment), unroll = 16-byte vectors per lane (the row stays in
// registers), block_k 0 and stages 1.  Candidates, the built-in choice first:
//   short rows (RMSNorm <= 512 vectors of 8, softmax <= 256): one wave per row;
//   longer rows up to 2048 vectors: a workgroup per row at 4 and at 8 waves
//   (8 first for softmax rows from 512 vectors and for RMSNorm rows above
//   1024 -- measured on [16384, 8192]: masked softmax 168.9 -> 162.0 us,
//   residual+RMSNorm equal; at 16384 columns 174.2 -> 171.8 and 136.5 ->
//   128.0 us; softmax at 3072 columns takes 4 waves first, 164.6 against
//   178.3 us);
//   2049 to 8192 vectors (up to 65536 columns): 16 waves first, then 8 (the row
//   still fits in registers: measured at 32768 columns residual+RMSNorm 478 ->
//   136 us and masked softmax 621 -> 184 us against the generic kernel, at
//   65536 columns 491 -> 176 and 622 -> 238 us, [rows, cols] of 2^27 elements);
//   8193 to 16384 vectors (up to 131072 columns): 16 waves, 16 vectors per
//   lane as packed bf16 (num_warps 16, unroll 16);
//   cols % 8 != 0 or longer rows: the generic kernel.
int row_vpt(int nvec, int lanes) {
  for (int v : {1, 2, 4, 8, 16})
    if (lanes * v >= nvec) return v;
  return 0;
}

int row_configs(bool softmax, int rows, int cols, pk_config *out, int cap) {
  if (rows <= 0 || cols <= 0) return 0;
  pk_config c[2];
  int n = 0;
  const int nvec = cols / 8;
  if (cols % 8 == 0 && nvec <= (softmax ? 256 : 512)) {
    c[n++] = pk_config{4, cols, 0, 4, 8, row_vpt(nvec, 64), 1};
  } else if (cols % 8 == 0 && nvec <= 2048) {
    // 4 waves: at least 4 vectors per lane for RMSNorm (the kernel's
    // instantiations), 2 for softmax
    const pk_config w4{1, cols, 0, 4, 8, std::max(softmax ? 2 : 4, row_vpt(nvec, 256)), 1};
    const pk_config w8{1, cols, 0, 8, 8, std::max(softmax ? 1 : 2, row_vpt(nvec, 512)), 1};
    // 8 waves first above 1024 vectors, and for softmax from 512 (3072
    // columns: 4 waves 164.6 against 178.3 us; 4096 a tie; 5120: 8 waves 164.2
    // against 170.6 us; 2^27-element problems)
    const bool eight_first = (softmax && nvec >= 512) || nvec > 1024;
    c[n++] = eight_first ? w8 : w4;
    c[n++] = eight_first ? w4 : w8;
  } else if (cols % 8 == 0 && nvec <= 8192) {
    // up to 65536 columns: 16 waves (a 1024-thread workgroup) with 4 or 8
    // vectors per lane first, 8 waves with 8 or 16 second
    c[n++] = pk_config{1, cols, 0, 16, 8, std::max(4, row_vpt(nvec, 1024)), 1};
    c[n++] = pk_config{1, cols, 0, 8, 8, std::max(8, row_vpt(nvec, 512)), 1};
  } else if (cols % 8 == 0 && nvec <= kPackedLanes * kPackedVpt) {
    // up to 131072 columns: 16 waves, 16 vectors per lane held as packed bf16
    c[n++] = pk_config{1, cols, 0, kPackedWaves, 8, kPackedVpt, 1};
  } else {
    c[n++] = pk_config{1, cols, 0, 4, 1, 1, 1};
  }
  for (int i = 0; i < n && i < cap; ++i) out[i] = c[i];
  return n;
}

bool row_config_listed(bool softmax, int rows, int cols, const pk_config &want) {
  pk_config c[2];
  const int n = row_configs(softmax, rows, cols, c, 2);
  for (int i = 0; i < n; ++i)
    if (std::memcmp(&c[i], &want, sizeof want) == 0) return true;
  return false;
}

// Launch the kernel a listed config names (vec: the operands are 16-byte
// aligned; a vector config needs that).
template <bool RESID>
int rmsnorm_run(const RowArgs &a, const pk_config &c, hipStream_t st) {
  if (c.vector_width == 1) {
    rmsnorm_generic_kernel<RESID><<<a.rows, kBlock, 0, st>>>(a);
    return PK_OK;
  }
  const unsigned rows = (unsigned)a.rows;
  if (c.block_m == 4) {
    const dim3 grid(rows / 4 + (rows % 4 != 0));
    switch (c.unroll) {
      case 1: rmsnorm_vec_kernel<1, 1, RESID><<<grid, kBlock, 0, st>>>(a); return PK_OK;
      case 2: rmsnorm_vec_kernel<1, 2, RESID><<<grid, kBlock, 0, st>>>(a); return PK_OK;
      case 4: rmsnorm_vec_kernel<1, 4, RESID><<<grid, kBlock, 0, st>>>(a); return PK_OK;
      case 8: rmsnorm_vec_kernel<1, 8, RESID><<<grid, kBlock, 0, st>>>(a); return PK_OK;
    }
  } else if (c.num_warps == 4) {
    switch (c.unroll) {
      case 4: rmsnorm_vec_kernel<4, 4, RESID><<<rows, 256, 0, st>>>(a); return PK_OK;
      case 8: rmsnorm_vec_kernel<4, 8, RESID><<<rows, 256, 0, st>>>(a); return PK_OK;
    }
  } else if (c.num_warps == 8) {
    switch (c.unroll) {
      case 2: rmsnorm_vec_kernel<8, 2, RESID><<<rows, 512, 0, st>>>(a); return PK_OK;
      case 4: rmsnorm_vec_kernel<8, 4, RESID><<<rows, 512, 0, st>>>(a); return PK_OK;
      case 8: rmsnorm_vec_kernel<8, 8, RESID><<<rows, 512, 0, st>>>(a); return PK_OK;
      case 16: rmsnorm_vec_kernel<8, 16, RESID><<<rows, 512, 0, st>>>(a); return PK_OK;
    }
  } else if (c.num_warps == 16) {
    switch (c.unroll) {
      case 4: rmsnorm_vec_kernel<16, 4, RESID><<<rows, 1024, 0, st>>>(a); return PK_OK;
      case 8: rmsnorm_vec_kernel<16, 8, RESID><<<rows, 1024, 0, st>>>(a); return PK_OK;
      case 16: rmsnorm_packed_kernel<RESID><<<rows, kPackedLanes, 0, st>>>(a); return PK_OK;
    }
  }
  set_error("rmsnorm: config {%d, %d, %d, %d, %d, %d, %d} has no kernel", c.block_m, c.block_n, c.block_k,
            c.num_warps, c.vector_width, c.unroll, c.shared_memory_stages);
  return PK_ERR_UNSUPPORTED;
}

template <int MODE>
int softmax_run(const RowArgs &a, const pk_config &c, hipStream_t st) {
  if (c.vector_width == 1) {
    softmax_generic_kernel<MODE><<<a.rows, kBlock, 0, st>>>(a);
    return PK_OK;
  }
  const unsigned rows = (unsigned)a.rows;
  if (c.block_m == 4) {
    const dim3 grid(rows / 4 + (rows % 4 != 0));
    switch (c.unroll) {
      case 1: softmax_vec_kernel<1, 1, MODE><<<grid, kBlock, 0, st>>>(a); return PK_OK;
      case 2: softmax_vec_kernel<1, 2, MODE><<<grid, kBlock, 0, st>>>(a); return PK_OK;
      case 4: softmax_vec_kernel<1, 4, MODE><<<grid, kBlock, 0, st>>>(a); return PK_OK;
    }
  } else if (c.num_warps == 4) {
    switch (c.unroll) {
      case 2: softmax_vec_kernel<4, 2, MODE><<<rows, 256, 0, st>>>(a); return PK_OK;
      case 4: softmax_vec_kernel<4, 4, MODE><<<rows, 256, 0, st>>>(a); return PK_OK;
      case 8: softmax_vec_kernel<4, 8, MODE><<<rows, 256, 0, st>>>(a); return PK_OK;
    }
  } else if (c.num_warps == 8) {
    switch (c.unroll) {
      case 1: softmax_vec_kernel<8, 1, MODE><<<rows, 512, 0, st>>>(a); return PK_OK;
      case 2: softmax_vec_kernel<8, 2, MODE><<<rows, 512, 0, st>>>(a); return PK_OK;
      case 4: softmax_vec_kernel<8, 4, MODE><<<rows, 512, 0, st>>>(a); return PK_OK;
      case 8: softmax_vec_kernel<8, 8, MODE><<<rows, 512, 0, st>>>(a); return PK_OK;
      case 16: softmax_vec_kernel<8, 16, MODE><<<rows, 512, 0, st>>>(a); return PK_OK;
    }
  } else if (c.num_warps == 16) {
    switch (c.unroll) {
      case 4: softmax_vec_kernel<16, 4, MODE><<<rows, 1024, 0, st>>>(a); return PK_OK;
      case 8: softmax_vec_kernel<16, 8, MODE><<<rows, 1024, 0, st>>>(a); return PK_OK;
      case 16: softmax_packed_kernel<MODE><<<rows, kPackedLanes, 0, st>>>(a); return PK_OK;
    }
  }
  set_error("softmax: config {%d, %d, %d, %d, %d, %d, %d} has no kernel", c.block_m, c.block_n, c.block_k,
            c.num_warps, c.vector_width, c.unroll, c.shared_memory_stages);
  return PK_ERR_UNSUPPORTED;
}

// cfg null: the built-in choice (the first candidate, or the generic kernel
// when the operands are not 16-byte aligned); otherwise a listed config, which
// must be the generic one when they are not.
template <bool RESID>
int rmsnorm_dispatch(const uint16_t *x, const uint16_t *r, const uint16_t *w, uint16_t *y, int rows, int cols,
                     float eps, const pk_config *cfg, hipStream_t st, const char *name) {
  PK_CHECK_ARG(x && y && (!RESID || r), "%s: null tensor pointer", name);
  PK_CHECK_ARG(rows >= 0 && cols > 0, "%s: invalid shape rows=%d cols=%d", name, rows, cols);
  PK_CHECK_ARG(!cfg || row_config_listed(false, std::max(rows, 1), cols, *cfg),
               "%s: config {%d, %d, %d, %d, %d, %d, %d} is not a row config for cols=%d", name,
               cfg ? cfg->block_m : 0, cfg ? cfg->block_n : 0, cfg ? cfg->block_k : 0, cfg ? cfg->num_warps : 0,
               cfg ? cfg->vector_width : 0, cfg ? cfg->unroll : 0, cfg ? cfg->shared_memory_stages : 0, cols);
  const bool aligned = aligned16(x) && aligned16(y) && (!RESID || aligned16(r)) && (!w || aligned16(w));
  if (cfg && cfg->vector_width == 8 && !aligned) {
    set_error("%s: the vector config needs 16-byte aligned x, r, gamma and out", name);
    return PK_ERR_UNSUPPORTED;
  }
  if (rows == 0) return PK_OK;
  const RowArgs a{x, RESID ? r : nullptr, w, y, rows, cols, 1.0f / (float)cols, eps};
  pk_config c;
  if (cfg) {
    c = *cfg;
  } else {
    row_configs(false, rows, cols, &c, 1);
    if (!aligned) c = pk_config{1, cols, 0, 4, 1, 1, 1};
  }
  int rc = rmsnorm_run<RESID>(a, c, st);
  if (rc) return rc;
  PK_LAUNCH_CHECK(name);
  return PK_OK;
}

template <int MODE>
int softmax_dispatch(const void *in, const uint16_t *mask, uint16_t *y, int rows, int cols, const pk_config *cfg,
                     hipStream_t st, const char *name) {
  PK_CHECK_ARG(in && y && (MODE == 0 || mask), "%s: null tensor pointer", name);
  PK_CHECK_ARG(rows >= 0 && cols > 0, "%s: invalid shape rows=%d cols=%d", name, rows, cols);
  PK_CHECK_ARG(!cfg || row_config_listed(true, std::max(rows, 1), cols, *cfg),
               "%s: config {%d, %d, %d, %d, %d, %d, %d} is not a row config for cols=%d", name,
               cfg ? cfg->block_m : 0, cfg ? cfg->block_n : 0, cfg ? cfg->block_k : 0, cfg ? cfg->num_warps : 0,
               cfg ? cfg->vector_width : 0, cfg ? cfg->unroll : 0, cfg ? cfg->shared_memory_stages : 0, cols);
  const bool aligned = aligned16(in) && aligned16(y) && (MODE == 0 || aligned16(mask));
  if (cfg && cfg->vector_width == 8 && !aligned) {
    set_error("%s: the vector config needs 16-byte aligned input, mask and out", name);
    return PK_ERR_UNSUPPORTED;
  }
  if (rows == 0) return PK_OK;
  const RowArgs a{in, MODE == 0 ? nullptr : mask, nullptr, y, rows, cols, 0.f, 0.f};
  pk_config c;
  if (cfg) {
    c = *cfg;
  } else {
    row_configs(true, rows, cols, &c, 1);
    if (!aligned) c = pk_config{1, cols, 0, 4, 1, 1, 1};
  }
  int rc = softmax_run<MODE>(a, c, st);
  if (rc) return rc;
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
  return rmsnorm_dispatch<false>(x, nullptr, w, y, rows, cols, eps, nullptr, st, "rmsnorm");
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

// The built-in choice for 16-byte aligned operands (the first candidate).
bool rmsnorm_config(int rows, int cols, pk_config *out) { return row_configs(false, rows, cols, out, 1) > 0; }
bool softmax_config(int rows, int cols, pk_config *out) { return row_configs(true, rows, cols, out, 1) > 0; }
int rmsnorm_configs(int rows, int cols, pk_config *out, int cap) { return row_configs(false, rows, cols, out, cap); }
int softmax_configs(int rows, int cols, pk_config *out, int cap) { return row_configs(true, rows, cols, out, cap); }

}  // namespace pk

using namespace pk;

extern "C" {

int launch_rmsnorm(const uint16_t *input, const uint16_t *weight, uint16_t *output, int rows,
                   int cols, float eps, void *stream) {
  return rmsnorm_dispatch<false>(input, nullptr, weight, output, rows, cols, eps, nullptr,
                                 (hipStream_t)stream, "launch_rmsnorm");
}

int launch_fused_residual_rmsnorm(const uint16_t *x, const uint16_t *r, const uint16_t *gamma,
                                  uint16_t *out, int rows, int cols, float eps, void *stream) {
  return rmsnorm_dispatch<true>(x, r, gamma, out, rows, cols, eps, nullptr, (hipStream_t)stream,
                                "launch_fused_residual_rmsnorm");
}

int pk_fused_residual_rmsnorm_config(const uint16_t *x, const uint16_t *r, const uint16_t *gamma, uint16_t *out,
                                     int rows, int cols, float eps, const pk_config *cfg, void *stream) {
  return rmsnorm_dispatch<true>(x, r, gamma, out, rows, cols, eps, cfg, (hipStream_t)stream,
                                "pk_fused_residual_rmsnorm_config");
}

int launch_softmax(const uint16_t *input, uint16_t *output, int rows, int cols, void *stream) {
  return softmax_dispatch<0>(input, nullptr, output, rows, cols, nullptr, (hipStream_t)stream,
                             "launch_softmax");
}

int launch_fused_softmax_mask(const float *logits, const uint16_t *mask, uint16_t *out, int rows,
                              int cols, void *stream) {
  return softmax_dispatch<1>(logits, mask, out, rows, cols, nullptr, (hipStream_t)stream,
                             "launch_fused_softmax_mask");
}

int pk_fused_softmax_mask_config(const float *logits, const uint16_t *mask, uint16_t *out, int rows, int cols,
                                 const pk_config *cfg, void *stream) {
  return softmax_dispatch<1>(logits, mask, out, rows, cols, cfg, (hipStream_t)stream,
                             "pk_fused_softmax_mask_config");
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
