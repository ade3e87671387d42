// naive.hip -- naive device implementations of every op, used as the golden
// of the autotuner's correctness gate, plus the device-side parity metrics.
//
// One thread per output element (per row for the row-wise ops and attention),
// each computing the reference's formula in the reference's own order:
//   matmul      c = bf16(sum_k a*b), k sequential, multiply then add
//               (kernels/cpu/cpu_reference.cpp:64-78)
//   bias/GELU   bf16(gelu(bf16(bf16(c) + bias))),
//               gelu(x) = (0.5x)(1 + (float)erf((double)(x * 0.70710678f)))
//               (cpu_reference.cpp:46-55, 92-105)
//   residual    bf16(f32(bf16(bf16(c) + bias)) + f32(r))  (golden.py:48-55)
//   int8        c = bf16(sum_k a * (f32(wq) * scale[n]))  (matmul_quant.cpp:169-204)
//   rmsnorm     ss sequential; rms = sqrt(ss * (1/cols) + eps); bf16((x/rms)*w)
//               (cpu_reference.cpp:16-44); residual form on bf16(x + r)
//   softmax     z = bf16(bf16(x) + mask), max seeded from z[0], sequential sum,
//               y = bf16(exp(z - m) * (1/sum))  (cpu_reference.cpp:107-128)
//   attention   attention.cpp:95-163 (score after the dot, causal offset
//               S_kv - S_q + i, PV then * 1/sum)
// The __f*_rn intrinsics keep every multiply and add separately rounded (no
// contraction into FMA).  These kernels are slow on purpose; nothing on the
// measured path calls them.
#include <algorithm>
#include <cmath>

#include "pk_common.hpp"

namespace pk {
namespace {

constexpr int kThreads = 256;

__device__ __forceinline__ float bfv(uint16_t b) { return bf2f(b); }
__device__ __forceinline__ float rbf(float x) { return bf2f(f2bf(x)); }

__device__ __forceinline__ float gelu_ref(float x) {
  const float h = __fmul_rn(0.5f, x);
  const float t = __fmul_rn(x, 0.70710678f);
  const float e = (float)erf((double)t);
  return __fmul_rn(h, __fadd_rn(1.0f, e));
}

// epi: 0 none, 1 bias + GELU, 2 bias (optional) + residual, 3 residual.
__global__ __launch_bounds__(kThreads) void naive_matmul_kernel(int epi, const uint16_t *__restrict__ A,
                                                                const uint16_t *__restrict__ B,
                                                                uint16_t *__restrict__ C,
                                                                const uint16_t *__restrict__ bias,
                                                                const uint16_t *__restrict__ R, int M, int N,
                                                                int K) {
  const int64_t idx = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (idx >= (int64_t)M * N) return;
  const int m = (int)(idx / N), n = (int)(idx % N);
  const uint16_t *a = A + (size_t)m * K;
  float acc = 0.0f;
  for (int k = 0; k < K; ++k) acc = __fadd_rn(acc, __fmul_rn(bfv(a[k]), bfv(B[(size_t)k * N + n])));
  float c = rbf(acc);
  if (epi == 1) {
    c = rbf(gelu_ref(rbf(__fadd_rn(c, bfv(bias[n])))));
  } else if (epi == 2) {
    if (bias) c = rbf(__fadd_rn(c, bfv(bias[n])));
    c = rbf(__fadd_rn(c, bfv(R[idx])));
  } else if (epi == 3) {
    c = rbf(__fadd_rn(c, bfv(R[idx])));
  }
  C[idx] = (uint16_t)f2bf(c);
}

// epi: 0 none, 1 GELU, 2 residual.
__global__ __launch_bounds__(kThreads) void naive_matmul_int8_kernel(int epi, const uint16_t *__restrict__ A,
                                                                     const int8_t *__restrict__ W,
                                                                     const float *__restrict__ scale,
                                                                     uint16_t *__restrict__ C,
                                                                     const uint16_t *__restrict__ R, int M,
                                                                     int N, int K) {
  const int64_t idx = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (idx >= (int64_t)M * N) return;
  const int m = (int)(idx / N), n = (int)(idx % N);
  const uint16_t *a = A + (size_t)m * K;
  const float s = scale[n];
  float acc = 0.0f;
  for (int k = 0; k < K; ++k)
    acc = __fadd_rn(acc, __fmul_rn(bfv(a[k]), __fmul_rn((float)W[(size_t)k * N + n], s)));
  float c = rbf(acc);
  if (epi == 1) c = rbf(gelu_ref(c));
  else if (epi == 2) c = rbf(__fadd_rn(c, bfv(R[idx])));
  C[idx] = (uint16_t)f2bf(c);
}

__global__ __launch_bounds__(kThreads) void naive_rmsnorm_kernel(const uint16_t *__restrict__ x,
                                                                 const uint16_t *__restrict__ r,
                                                                 const uint16_t *__restrict__ w,
                                                                 uint16_t *__restrict__ y, int rows, int cols,
                                                                 float eps) {
  const int row = blockIdx.x * kThreads + threadIdx.x;
  if (row >= rows) return;
  const size_t base = (size_t)row * cols;
  auto val = [&](int c) { return r ? rbf(__fadd_rn(bfv(x[base + c]), bfv(r[base + c]))) : bfv(x[base + c]); };
  float ss = 0.0f;
  for (int c = 0; c < cols; ++c) {
    const float v = val(c);
    ss = __fadd_rn(ss, __fmul_rn(v, v));
  }
  const float inv_cols = __fdiv_rn(1.0f, (float)cols);
  const float rms = __fsqrt_rn(__fadd_rn(__fmul_rn(ss, inv_cols), eps));
  for (int c = 0; c < cols; ++c) {
    float o = __fdiv_rn(val(c), rms);
    if (w) o = __fmul_rn(o, bfv(w[c]));
    y[base + c] = (uint16_t)f2bf(o);
  }
}

__global__ __launch_bounds__(kThreads) void naive_softmax_mask_kernel(const float *__restrict__ x,
                                                                      const uint16_t *__restrict__ mask,
                                                                      uint16_t *__restrict__ y, int rows,
                                                                      int cols) {
  const int row = blockIdx.x * kThreads + threadIdx.x;
  if (row >= rows) return;
  const size_t base = (size_t)row * cols;
  auto z = [&](int c) { return rbf(__fadd_rn(rbf(x[base + c]), bfv(mask[base + c]))); };
  float m = z(0);
  for (int c = 1; c < cols; ++c) m = fmaxf(m, z(c));
  float s = 0.0f;
  for (int c = 0; c < cols; ++c) s = __fadd_rn(s, expf(__fsub_rn(z(c), m)));
  const float inv = __fdiv_rn(1.0f, s);
  for (int c = 0; c < cols; ++c) y[base + c] = (uint16_t)f2bf(__fmul_rn(expf(__fsub_rn(z(c), m)), inv));
}

// Head dims up to the library's 1024; a thread keeps 256 output dims in
// registers and takes the key loop again for each further 256 (every output
// element still sums its keys in order).
constexpr int kMaxD = 1024, kChunkD = 256;

__global__ __launch_bounds__(64) void naive_attention_kernel(const uint16_t *__restrict__ Q,
                                                             const uint16_t *__restrict__ K,
                                                             const uint16_t *__restrict__ V,
                                                             uint16_t *__restrict__ O, int BH, int S_q, int S_kv,
                                                             int kv_stride, int D, float scale, int causal) {
  const int64_t row = (int64_t)blockIdx.x * 64 + threadIdx.x;
  if (row >= (int64_t)BH * S_q) return;
  const int64_t bh = row / S_q;
  const int i = (int)(row % S_q);
  const uint16_t *q = Q + row * D;
  const uint16_t *kb = K + bh * kv_stride * (int64_t)D;
  const uint16_t *vb = V + bh * kv_stride * (int64_t)D;
  const int limit = causal ? S_kv - S_q + i : S_kv - 1;
  auto score = [&](int j) {
    float d = 0.0f;
    for (int t = 0; t < D; ++t) d = __fadd_rn(d, __fmul_rn(bfv(q[t]), bfv(kb[(int64_t)j * D + t])));
    return __fmul_rn(d, scale);
  };
  float m = -INFINITY;
  for (int j = 0; j <= limit && j < S_kv; ++j) m = fmaxf(m, score(j));
  for (int c0 = 0; c0 < D; c0 += kChunkD) {
    const int cn = min(kChunkD, D - c0);
    float o[kChunkD];
    for (int t = 0; t < cn; ++t) o[t] = 0.0f;
    float sum = 0.0f;  // the same sum on every pass
    for (int j = 0; j <= limit && j < S_kv; ++j) {
      const float w = expf(__fsub_rn(score(j), m));
      sum = __fadd_rn(sum, w);
      for (int t = 0; t < cn; ++t) o[t] = __fadd_rn(o[t], __fmul_rn(w, bfv(vb[(int64_t)j * D + c0 + t])));
    }
    const float inv = __fdiv_rn(1.0f, sum);
    for (int t = 0; t < cn; ++t) O[row * D + c0 + t] = (uint16_t)f2bf(__fmul_rn(o[t], inv));
  }
}

// ---- parity metrics -----------------------------------------------------------
// Pass 1 per block: sum g, sum w, sum g^2, sum w^2, sum g*w, max rel, equal
// count, NaN flag.  Pass 2: centred sums for the Pearson correlation.
constexpr int kMetricBlocks = 1024;
constexpr int kP1 = 8, kP2 = 3;

__device__ __forceinline__ double block_sum(double v, double *red) {
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) red[wid] = v;
  __syncthreads();
  double t = 0.0;
  if (threadIdx.x == 0)
    for (int i = 0; i < kThreads / 64; ++i) t += red[i];
  return t;
}

__device__ __forceinline__ double block_max(double v, double *red) {
  for (int off = 32; off >= 1; off >>= 1) v = fmax(v, __shfl_xor(v, off, 64));
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) red[wid] = v;
  __syncthreads();
  double t = 0.0;
  if (threadIdx.x == 0)
    for (int i = 0; i < kThreads / 64; ++i) t = fmax(t, red[i]);
  return t;
}

__global__ __launch_bounds__(kThreads) void metrics_pass1(const uint16_t *__restrict__ g,
                                                          const uint16_t *__restrict__ w, int64_t n,
                                                          double *__restrict__ part) {
  __shared__ double red[kThreads / 64];
  double sg = 0, sw = 0, sgg = 0, sww = 0, sgw = 0, mrel = 0, eq = 0, nan = 0;
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += (int64_t)gridDim.x * kThreads) {
    const double a = bf2f(g[i]), b = bf2f(w[i]);
    if (a != a || b != b) {
      nan = 1.0;
      continue;
    }
    sg += a;
    sw += b;
    sgg += a * a;
    sww += b * b;
    sgw += a * b;
    mrel = fmax(mrel, fabs(a - b) / (fabs(b) + 1e-6));
    eq += (g[i] == w[i]) ? 1.0 : 0.0;
  }
  const double vals[kP1] = {sg, sw, sgg, sww, sgw, mrel, eq, nan};
  for (int q = 0; q < kP1; ++q) {
    const double t = (q == 5 || q == 7) ? block_max(vals[q], red) : block_sum(vals[q], red);
    if (threadIdx.x == 0) part[(size_t)blockIdx.x * kP1 + q] = t;
  }
}

__global__ __launch_bounds__(kThreads) void metrics_pass2(const uint16_t *__restrict__ g,
                                                          const uint16_t *__restrict__ w, int64_t n, double mg,
                                                          double mw, double *__restrict__ part) {
  __shared__ double red[kThreads / 64];
  double cgg = 0, cww = 0, cgw = 0;
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += (int64_t)gridDim.x * kThreads) {
    const double a = bf2f(g[i]) - mg, b = bf2f(w[i]) - mw;
    cgg += a * a;
    cww += b * b;
    cgw += a * b;
  }
  const double vals[kP2] = {cgg, cww, cgw};
  for (int q = 0; q < kP2; ++q) {
    const double t = block_sum(vals[q], red);
    if (threadIdx.x == 0) part[(size_t)blockIdx.x * kP2 + q] = t;
  }
}

int grid1d(int64_t n, int per_block = kThreads) { return (int)((n + per_block - 1) / per_block); }

// ---- the autotuner's error-model gate ---------------------------------------
// An output of a GEMM-class op passes when it is what the reference's epilogue
// gives for SOME fp32 accumulation of the same products.  Any order of an fp32
// sum of K terms lies within K 2^-24 sum|p| of the exact sum (the classic
// gamma_K bound), two such sums within twice that, so the accumulator t may be
// anywhere in S +- delta, delta = (K 2^-23 + extra) sum|p|, with S and sum|p|
// exact (fp64; bf16 x bf16 and bf16 x int8 x fp32 products are exact there).
// RNE is monotone, so bf16(t) lies between the codes of the interval's ends;
// bias and residual adds are non-decreasing in t, GELU decreases below its
// minimum at x ~ -0.7518 and increases above, so the epilogue maps that code
// range onto [lo, hi] computed from the ends -- by a scan of every code when
// the range is short, else from the ends plus GELU's minimum where the range
// straddles it.  A wrong index, sign, dropped term or dropped bias moves most
// outputs outside; summation order alone never does.
struct GateArgs {
  int mode;  // 0: bf16 x bf16, 1: bf16 x int8 (per-column scale)
  int epi;   // bf16: 0 none, 1 bias + GELU, 2 bias (optional) + residual, 3 residual;
             // int8: 0 none, 1 GELU, 2 residual
  const uint16_t *A;
  const uint16_t *B;
  const int8_t *Wq;
  const float *scale;
  const uint16_t *bias;
  const uint16_t *R;
  const uint16_t *got;
  const uint16_t *tab;
  int M, N, K;
  double rel;  // K 2^-23 (+ extra) per unit of sum|p|
  unsigned long long *bad;
};

__device__ __forceinline__ int bf_key(uint32_t b) { return (b & 0x8000u) ? -(int)(b & 0x7FFFu) : (int)b; }
__device__ __forceinline__ uint32_t bf_from_key(int k) { return k >= 0 ? (uint32_t)k : (0x8000u | (uint32_t)(-k)); }

// Lower (upper) bound on bf16(t) over every fp32 t >= x (t <= x): the code of
// the largest fp32 value <= x (smallest >= x).
__device__ __forceinline__ uint32_t bf_bound(double x, bool upper) {
  float f = (float)x;
  if (upper && (double)f < x) f = nextafterf(f, INFINITY);
  if (!upper && (double)f > x) f = nextafterf(f, -INFINITY);
  return f2bf(f);
}

__device__ __forceinline__ float gate_gelu(uint32_t u, const uint16_t *tab) { return bf2f(gelu_bits(u, tab)); }

__global__ __launch_bounds__(kThreads) void gate_kernel(GateArgs g) {
  const int64_t idx = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  bool bad = false;
  if (idx < (int64_t)g.M * g.N) {
    const int m = (int)(idx / g.N), n = (int)(idx % g.N);
    const uint16_t *a = g.A + (size_t)m * g.K;
    double S = 0.0, T = 0.0;
    if (g.mode == 0) {
      for (int k = 0; k < g.K; ++k) {
        const double p = (double)bf2f(a[k]) * (double)bf2f(g.B[(size_t)k * g.N + n]);
        S += p;
        T += fabs(p);
      }
    } else {
      const double sc = (double)g.scale[n];
      for (int k = 0; k < g.K; ++k) {
        const double p = (double)bf2f(a[k]) * ((double)g.Wq[(size_t)k * g.N + n] * sc);
        S += p;
        T += fabs(p);
      }
    }
    const double delta = g.rel * T * (1.0 + 0x1p-20) + g.K * 0x1p-149;
    uint32_t clo = bf_bound(S - delta, false), chi = bf_bound(S + delta, true);
    const float r = g.R ? bf2f(g.R[idx]) : 0.0f;
    const bool gelu = g.epi == 1;
    float lo, hi;
    if (gelu) {
      uint32_t ulo = clo, uhi = chi;
      if (g.mode == 0) {  // u = bf16(bf16(t) + bias)
        const float b = bf2f(g.bias[n]);
        ulo = f2bf(bf2f(clo) + b);
        uhi = f2bf(bf2f(chi) + b);
      }
      const int kl = bf_key(ulo), kh = bf_key(uhi);
      lo = INFINITY;
      hi = -INFINITY;
      if (kh - kl <= 512) {
        for (int kk = kl; kk <= kh; ++kk) {
          const float v = gate_gelu(bf_from_key(kk), g.tab);
          lo = fminf(lo, v);
          hi = fmaxf(hi, v);
        }
      } else {
        const float vl = gate_gelu(ulo, g.tab), vh = gate_gelu(uhi, g.tab);
        lo = fminf(vl, vh);
        hi = fmaxf(vl, vh);
        if (bf2f(ulo) < -0.5f && bf2f(uhi) > -1.0f)  // the minimum lies in [-1, -0.5]
          for (uint32_t c = 0xBF00u; c <= 0xBF80u; ++c) lo = fminf(lo, gate_gelu(c, g.tab));
      }
    } else {
      auto f = [&](uint32_t c) -> float {
        float v = bf2f(c);
        if (g.mode == 0 && g.epi == 2 && g.bias) v = bf2f(f2bf(v + bf2f(g.bias[n])));
        if (g.R) v = bf2f(f2bf(v + r));
        return v;
      };
      lo = f(clo);
      hi = f(chi);
    }
    const float got = bf2f(g.got[idx]);
    bad = !(got >= lo && got <= hi);
  }
  const unsigned long long votes = __ballot(bad);
  if ((threadIdx.x & 63) == 0 && votes) atomicAdd(g.bad, (unsigned long long)__popcll(votes));
}

int run_gate(GateArgs g, unsigned long long *bad_host, hipStream_t st) {
  *bad_host = 0;
  if ((int64_t)g.M * g.N == 0) return PK_OK;
  if (g.epi == 1) {
    int rc = gelu_table(&g.tab);
    if (rc) return rc;
  }
  unsigned long long *d = nullptr;
  PK_HIP(hipMalloc(&d, sizeof *d));
  hipError_t e = hipMemsetAsync(d, 0, sizeof *d, st);
  g.bad = d;
  if (e == hipSuccess) {
    gate_kernel<<<grid1d((int64_t)g.M * g.N), kThreads, 0, st>>>(g);
    e = hipGetLastError();
  }
  if (e == hipSuccess) e = hipMemcpyAsync(bad_host, d, sizeof *d, hipMemcpyDeviceToHost, st);
  if (e == hipSuccess) e = hipStreamSynchronize(st);
  (void)hipFree(d);
  return e == hipSuccess ? PK_OK : hip_fail(e, "error-model gate");
}


}  // namespace
}  // namespace pk

using namespace pk;

extern "C" {

int pk_naive_matmul(int epi, const uint16_t *A, const uint16_t *B, uint16_t *C, const uint16_t *bias,
                    const uint16_t *R, int M, int N, int K, void *stream) {
  PK_CHECK_ARG(A && B && C, "pk_naive_matmul: null tensor pointer");
  PK_CHECK_ARG(epi >= 0 && epi <= 3, "pk_naive_matmul: epilogue %d not in 0..3", epi);
  PK_CHECK_ARG((epi != 1 || bias) && (epi < 2 || R), "pk_naive_matmul: epilogue operand missing");
  PK_CHECK_ARG(M >= 0 && N >= 0 && K >= 0, "pk_naive_matmul: invalid shape");
  if ((int64_t)M * N == 0) return PK_OK;
  naive_matmul_kernel<<<grid1d((int64_t)M * N), kThreads, 0, (hipStream_t)stream>>>(epi, A, B, C, bias, R, M, N,
                                                                                     K);
  PK_LAUNCH_CHECK("naive_matmul_kernel");
  return PK_OK;
}

int pk_naive_matmul_int8(int epi, const uint16_t *A, const int8_t *Wq, const float *scale, uint16_t *C,
                         const uint16_t *R, int M, int N, int K, void *stream) {
  PK_CHECK_ARG(A && Wq && scale && C && (epi != 2 || R), "pk_naive_matmul_int8: null tensor pointer");
  PK_CHECK_ARG(epi >= 0 && epi <= 2, "pk_naive_matmul_int8: epilogue %d not in 0..2", epi);
  PK_CHECK_ARG(M >= 0 && N >= 0 && K >= 0, "pk_naive_matmul_int8: invalid shape");
  if ((int64_t)M * N == 0) return PK_OK;
  naive_matmul_int8_kernel<<<grid1d((int64_t)M * N), kThreads, 0, (hipStream_t)stream>>>(epi, A, Wq, scale, C, R,
                                                                                          M, N, K);
  PK_LAUNCH_CHECK("naive_matmul_int8_kernel");
  return PK_OK;
}

int pk_naive_rmsnorm(const uint16_t *x, const uint16_t *r, const uint16_t *gamma, uint16_t *out, int rows,
                     int cols, float eps, void *stream) {
  PK_CHECK_ARG(x && out, "pk_naive_rmsnorm: null tensor pointer");
  PK_CHECK_ARG(rows >= 0 && cols > 0, "pk_naive_rmsnorm: invalid shape");
  if (rows == 0) return PK_OK;
  naive_rmsnorm_kernel<<<grid1d(rows), kThreads, 0, (hipStream_t)stream>>>(x, r, gamma, out, rows, cols, eps);
  PK_LAUNCH_CHECK("naive_rmsnorm_kernel");
  return PK_OK;
}

int pk_naive_softmax_mask(const float *logits, const uint16_t *mask, uint16_t *out, int rows, int cols,
                          void *stream) {
  PK_CHECK_ARG(logits && mask && out, "pk_naive_softmax_mask: null tensor pointer");
  PK_CHECK_ARG(rows >= 0 && cols > 0, "pk_naive_softmax_mask: invalid shape");
  if (rows == 0) return PK_OK;
  naive_softmax_mask_kernel<<<grid1d(rows), kThreads, 0, (hipStream_t)stream>>>(logits, mask, out, rows, cols);
  PK_LAUNCH_CHECK("naive_softmax_mask_kernel");
  return PK_OK;
}

int pk_naive_attention(const uint16_t *Q, const uint16_t *K, const uint16_t *V, uint16_t *O, int BH, int S_q,
                       int S_kv, int kv_stride, int D, float scale, int causal, void *stream) {
  PK_CHECK_ARG(Q && K && V && O, "pk_naive_attention: null tensor pointer");
  PK_CHECK_ARG(BH >= 0 && S_q >= 0 && S_kv > 0 && kv_stride >= S_kv && D > 0 && D <= kMaxD,
               "pk_naive_attention: invalid shape");
  PK_CHECK_ARG(!causal || S_kv >= S_q, "pk_naive_attention: causal needs S_kv >= S_q");
  if ((int64_t)BH * S_q == 0) return PK_OK;
  naive_attention_kernel<<<grid1d((int64_t)BH * S_q, 64), 64, 0, (hipStream_t)stream>>>(Q, K, V, O, BH, S_q, S_kv,
                                                                                        kv_stride, D, scale, causal);
  PK_LAUNCH_CHECK("naive_attention_kernel");
  return PK_OK;
}

int pk_gate_matmul(int epi, const uint16_t *A, const uint16_t *B, const uint16_t *bias, const uint16_t *R,
                   const uint16_t *got, int M, int N, int K, double operand_ulps, unsigned long long *bad,
                   void *stream) {
  PK_CHECK_ARG(A && B && got && bad, "pk_gate_matmul: null argument");
  PK_CHECK_ARG(epi >= 0 && epi <= 3, "pk_gate_matmul: epilogue %d not in 0..3", epi);
  PK_CHECK_ARG((epi != 1 || bias) && (epi < 2 || R), "pk_gate_matmul: epilogue operand missing");
  PK_CHECK_ARG(M >= 0 && N >= 0 && K >= 0 && operand_ulps >= 0, "pk_gate_matmul: invalid argument");
  GateArgs g{0, epi, A, B, nullptr, nullptr, epi == 1 || epi == 2 ? bias : nullptr, epi >= 2 ? R : nullptr, got,
             nullptr, M, N, K, K * 0x1p-23 + operand_ulps * 0x1p-8, nullptr};
  return run_gate(g, bad, (hipStream_t)stream);
}

int pk_gate_matmul_int8(int epi, const uint16_t *A, const int8_t *Wq, const float *scale, const uint16_t *R,
                        const uint16_t *got, int M, int N, int K, unsigned long long *bad, void *stream) {
  PK_CHECK_ARG(A && Wq && scale && got && bad && (epi != 2 || R), "pk_gate_matmul_int8: null argument");
  PK_CHECK_ARG(epi >= 0 && epi <= 2, "pk_gate_matmul_int8: epilogue %d not in 0..2", epi);
  PK_CHECK_ARG(M >= 0 && N >= 0 && K >= 0, "pk_gate_matmul_int8: invalid shape");
  // the reference rounds w*scale and a*(w*scale) once each before the sum
  GateArgs g{1, epi, A, nullptr, Wq, scale, nullptr, epi == 2 ? R : nullptr, got, nullptr, M, N, K,
             (K + 2) * 0x1p-23, nullptr};
  return run_gate(g, bad, (hipStream_t)stream);
}

int pk_compare_bf16(const uint16_t *got, const uint16_t *want, long long n, double out[4], void *stream) {
  PK_CHECK_ARG(got && want && out && n >= 0, "pk_compare_bf16: invalid argument");
  if (n == 0) {
    out[0] = 1.0;
    out[1] = 0.0;
    out[2] = 1.0;
    out[3] = 1.0;
    return PK_OK;
  }
  hipStream_t st = (hipStream_t)stream;
  const int blocks = (int)std::min<int64_t>(kMetricBlocks, ((int64_t)n + kThreads - 1) / kThreads);
  double *part = nullptr;
  PK_HIP(hipMalloc(&part, (size_t)blocks * kP1 * sizeof(double)));
  double h1[kMetricBlocks * kP1], h2[kMetricBlocks * kP2];
  auto fail = [&](hipError_t e, const char *what) {
    (void)hipFree(part);
    return hip_fail(e, what);
  };
  metrics_pass1<<<blocks, kThreads, 0, st>>>(got, want, n, part);
  hipError_t e = hipGetLastError();
  if (e == hipSuccess) e = hipMemcpyAsync(h1, part, (size_t)blocks * kP1 * sizeof(double), hipMemcpyDeviceToHost, st);
  if (e == hipSuccess) e = hipStreamSynchronize(st);
  if (e != hipSuccess) return fail(e, "pk_compare_bf16 pass 1");
  double s[kP1] = {};
  for (int b = 0; b < blocks; ++b)
    for (int q = 0; q < kP1; ++q) {
      const double v = h1[(size_t)b * kP1 + q];
      s[q] = (q == 5 || q == 7) ? std::max(s[q], v) : s[q] + v;
    }
  const double nn = (double)n;
  metrics_pass2<<<blocks, kThreads, 0, st>>>(got, want, n, s[0] / nn, s[1] / nn, part);
  e = hipGetLastError();
  if (e == hipSuccess) e = hipMemcpyAsync(h2, part, (size_t)blocks * kP2 * sizeof(double), hipMemcpyDeviceToHost, st);
  if (e == hipSuccess) e = hipStreamSynchronize(st);
  if (e != hipSuccess) return fail(e, "pk_compare_bf16 pass 2");
  PK_HIP(hipFree(part));
  double c[kP2] = {};
  for (int b = 0; b < blocks; ++b)
    for (int q = 0; q < kP2; ++q) c[q] += h2[(size_t)b * kP2 + q];
  if (s[7] != 0.0) {  // a NaN on either side fails every metric
    out[0] = out[1] = out[2] = NAN;
    out[3] = s[6] / nn;
    return PK_OK;
  }
  const double nx = std::sqrt(s[2]), ny = std::sqrt(s[3]);
  out[0] = (nx * ny == 0.0) ? ((nx == 0.0 && ny == 0.0) ? 1.0 : 0.0) : s[4] / (nx * ny);
  out[1] = s[5];
  const double den = std::sqrt(c[0]) * std::sqrt(c[1]);
  out[2] = den == 0.0 ? (s[6] == nn ? 1.0 : 0.0) : c[2] / den;
  out[3] = s[6] / nn;
  return PK_OK;
}

}  // extern "C"
