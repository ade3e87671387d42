// rowwise_kernels.hpp -- the HBM-bound row kernels for gfx950 (bodies):
// RMSNorm / residual + RMSNorm and softmax / masked softmax, shared by the
// library (rowwise.hip, which wraps them as __global__ kernels) and by code
// objects the emitter instantiates at a tuned configuration
// (csrc/runtime/codegen.cpp).  Both compile this one source.
//
// One row per wave (short rows) or per block of NW = 4 or 8 waves (long rows),
// the row held in registers so every input byte is read from HBM exactly once;
// 16-byte vector loads/stores; wave64 shuffle reductions, then one LDS exchange
// across the block's waves.
#pragma once

#include "pk_common.hpp"
#include "rowwise_args.h"

namespace pk {

// Kernel arguments: struct pk_row_args of rowwise_args.h (host and device share it).
using RowArgs = pk_row_args;

namespace row {

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

// ---------------------------------------------------------------------------
// RMSNorm / residual + RMSNorm (vector path: cols % 8 == 0, 16-byte aligned).
// NW waves cooperate on one row in a block of NW * 64 threads (NW == 1: each
// wave owns a row, 4 rows per 256-thread block).  Each lane keeps VPT
// 8-element vectors of the row in registers.
// Arithmetic per kernels/cpu/cpu_reference.cpp:16-44: ss = sum x^2 (fp32),
// rms = sqrt(ss * (1/cols) + eps), y = bf16((x / rms) [* w]).  With a residual
// the normalised value is s = bf16(x + r) (tests/golden/golden.py:108-112).
// ---------------------------------------------------------------------------
template <int NW, int VPT, bool RESID>
__device__ __forceinline__ void rmsnorm_vec_body(const RowArgs &a) {
#pragma clang fp contract(off)
  const uint16_t *__restrict__ x = static_cast<const uint16_t *>(a.in);
  const uint16_t *__restrict__ r = a.aux;
  const uint16_t *__restrict__ w = a.gamma;
  uint16_t *__restrict__ y = a.out;
  const int rows = a.rows, cols = a.cols;
  const float inv_cols = a.inv_cols, eps = a.eps;
  __shared__ float red[NW];
  constexpr int kRowsPerBlock = (NW == 1) ? (kBlock / 64) : 1;
  constexpr int kLanes = NW * 64;
  const unsigned row = (NW == 1) ? (blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6)) : blockIdx.x;
  const int lane = (NW == 1) ? (threadIdx.x & 63) : threadIdx.x;
  if (row >= (unsigned)rows) return;  // uniform per row-group (NW == 1: per wave)
  const int nvec = cols >> 3;
  const size_t base = (size_t)row * cols;

  // Every load of the row (and residual) is issued before the first is
  // unpacked ([4096, 4096] + gamma 14.05 -> 13.55 us, residual + RMSNorm
  // [16384, 8192] 126.7 -> 124.1 us, bit-identical).
  U4 xw[VPT], rw[RESID ? VPT : 1];
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    const int c = lane + i * kLanes;
    if (c < nvec) {
      xw[i] = ld16_once(x + base + (size_t)c * 8);
      if constexpr (RESID) rw[i] = ld16_once(r + base + (size_t)c * 8);
    }
  }
  float v[VPT][8];
  float ss = 0.f;
  DivSpan span;  // magnitudes of the numerators (without a residual: the loaded words)
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    const int c = lane + i * kLanes;
    if (c < nvec) {
      unpack8(xw[i], v[i]);
      if constexpr (!RESID) {
        div_span_add(span, xw[i].x);
        div_span_add(span, xw[i].y);
        div_span_add(span, xw[i].z);
        div_span_add(span, xw[i].w);
      }
      if constexpr (RESID) {
        float rv[8];
        unpack8(rw[i], rv);
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
  if constexpr (RESID) {
#pragma unroll
    for (int i = 0; i < VPT; ++i)
      if (lane + i * kLanes < nvec)
#pragma unroll
        for (int e = 0; e < 8; ++e) ok &= div_elem_ok(v[i][e]);
  } else {
    ok &= div_span_ok(span);
  }
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
// row (the second from cache).  Column indices are unsigned so that stepping
// past a cols near INT32_MAX cannot wrap.
template <bool RESID>
__device__ __forceinline__ void rmsnorm_generic_body(const RowArgs &a) {
#pragma clang fp contract(off)
  const uint16_t *__restrict__ x = static_cast<const uint16_t *>(a.in);
  const uint16_t *__restrict__ r = a.aux;
  const uint16_t *__restrict__ w = a.gamma;
  uint16_t *__restrict__ y = a.out;
  const int cols = a.cols;
  const float inv_cols = a.inv_cols, eps = a.eps;
  __shared__ float red[kBlock / 64];
  const int row = blockIdx.x;
  const size_t base = (size_t)row * cols;
  float ss = 0.f;
  for (unsigned c = threadIdx.x; c < (unsigned)cols; c += kBlock) {
    float s = bf2f(x[base + c]);
    if constexpr (RESID) s = bf2f(f2bf(s + bf2f(r[base + c])));
    ss += s * s;
  }
  ss = group_sum<kBlock / 64>(ss, red);
  const float rms = sqrtf(ss * inv_cols + eps);
  for (unsigned c = threadIdx.x; c < (unsigned)cols; c += kBlock) {
    float s = bf2f(x[base + c]);
    if constexpr (RESID) s = bf2f(f2bf(s + bf2f(r[base + c])));
    float o = s / rms;
    if (w) o *= bf2f(w[c]);
    y[base + c] = (uint16_t)f2bf(o);
  }
}

// ---------------------------------------------------------------------------
// Softmax over the last axis.  MODE 0: bf16 input (kernels/cpu/cpu_reference.cpp:107-128);
// MODE 1: fp32 logits + bf16 additive mask, z = bf16(bf16(x) + mask)
// (tests/golden/golden.py:115-117).  m = max z, e = exp(z - m), y = bf16(e * (1/sum e)).
// ---------------------------------------------------------------------------
// The words of 8 consecutive inputs (MODE 0: 8 bf16 in a; MODE 1: 8 fp32 in
// a, b and 8 bf16 mask values in mk) and the softmax input z they give.
template <int MODE>
struct Z8Words {
  U4 a, b, mk;
};
template <int MODE>
__device__ __forceinline__ Z8Words<MODE> load_z8_words(const void *in, const uint16_t *mask, size_t off) {
  Z8Words<MODE> w;
  if constexpr (MODE == 0) {
    w.a = ld16_once(static_cast<const uint16_t *>(in) + off);
  } else {
    const float *xf = static_cast<const float *>(in) + off;
    w.a = ld16_once(xf);
    w.b = ld16_once(xf + 4);
    w.mk = ld16_once(mask + off);
  }
  return w;
}
template <int MODE>
__device__ __forceinline__ void z8_of(const Z8Words<MODE> &w, float (&z)[8]) {
#pragma clang fp contract(off)
  if constexpr (MODE == 0) {
    unpack8(w.a, z);
  } else {
    float m[8];
    unpack8(w.mk, m);
    const uint32_t raw[8] = {w.a.x, w.a.y, w.a.z, w.a.w, w.b.x, w.b.y, w.b.z, w.b.w};
#pragma unroll
    for (int e = 0; e < 8; ++e) z[e] = bf2f(f2bf(bf2f(f2bf(__uint_as_float(raw[e]))) + m[e]));
  }
}
template <int MODE>
__device__ __forceinline__ void load_z8(const void *in, const uint16_t *mask, size_t off,
                                        float (&z)[8]) {
  z8_of<MODE>(load_z8_words<MODE>(in, mask, off), z);
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
__device__ __forceinline__ void softmax_vec_body(const RowArgs &a) {
#pragma clang fp contract(off)
  const void *__restrict__ in = a.in;
  const uint16_t *__restrict__ mask = a.aux;
  uint16_t *__restrict__ y = a.out;
  const int rows = a.rows, cols = a.cols;
  __shared__ float red[NW];
  constexpr int kRowsPerBlock = (NW == 1) ? (kBlock / 64) : 1;
  constexpr int kLanes = NW * 64;
  const unsigned row = (NW == 1) ? (blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6)) : blockIdx.x;
  const int lane = (NW == 1) ? (threadIdx.x & 63) : threadIdx.x;
  if (row >= (unsigned)rows) return;
  const int nvec = cols >> 3;
  const size_t base = (size_t)row * cols;

  // every load of the row before the first conversion, as in rmsnorm_vec_body
  Z8Words<MODE> zw[VPT];
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    const int c = lane + i * kLanes;
    if (c < nvec) zw[i] = load_z8_words<MODE>(in, mask, base + (size_t)c * 8);
  }
  float z[VPT][8];
  float m = -INFINITY;
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    const int c = lane + i * kLanes;
    if (c < nvec) {
      z8_of<MODE>(zw[i], z[i]);
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
__device__ __forceinline__ void softmax_generic_body(const RowArgs &a) {
#pragma clang fp contract(off)
  const void *__restrict__ in = a.in;
  const uint16_t *__restrict__ mask = a.aux;
  uint16_t *__restrict__ y = a.out;
  const int cols = a.cols;
  __shared__ float red[kBlock / 64];
  const int row = blockIdx.x;
  const size_t base = (size_t)row * cols;
  float m = -INFINITY;
  for (unsigned c = threadIdx.x; c < (unsigned)cols; c += kBlock) m = fmaxf(m, load_z1<MODE>(in, mask, base + c));
  m = group_max<kBlock / 64>(m, red);
  float s = 0.f;
  for (unsigned c = threadIdx.x; c < (unsigned)cols; c += kBlock) s += expf(load_z1<MODE>(in, mask, base + c) - m);
  s = group_sum<kBlock / 64>(s, red);
  const float inv = 1.0f / s;
  for (unsigned c = threadIdx.x; c < (unsigned)cols; c += kBlock)
    y[base + c] = (uint16_t)f2bf(expf(load_z1<MODE>(in, mask, base + c) - m) * inv);
}

// ---------------------------------------------------------------------------
// Rows of up to kPackedLanes * kPackedVpt * 8 = 131072 columns (cols % 8 == 0,
// 16-byte aligned): one row per workgroup of 16 waves, each lane keeping its
// 16 vectors as packed bf16 -- the values both ops hold are bf16 (the rounded
// residual sum s, or x; the rounded masked logit z) -- so the row stays in 64
// registers and HBM is read once.  Softmax keeps half of its chunks in LDS
// (128 KiB) so that the exponentials' temporaries fit the 128 registers of a
// 1024-thread workgroup without spilling (vocabulary-length rows 2.9-3.4 ->
// 3.5-4.1 TB/s, bit-identical), and sums online while the row arrives (each
// lane's sum rescaled whenever its running max grows), so exp(z - m) is
// evaluated again only for the output (4.3-4.9 TB/s).  RMSNorm arithmetic as
// in the vector bodies.
// ---------------------------------------------------------------------------
constexpr int kPackedWaves = 16, kPackedLanes = kPackedWaves * 64, kPackedVpt = 16;

template <bool RESID>
__device__ __forceinline__ void rmsnorm_packed_body(const RowArgs &a) {
#pragma clang fp contract(off)
  const uint16_t *__restrict__ x = static_cast<const uint16_t *>(a.in);
  const uint16_t *__restrict__ r = a.aux;
  const uint16_t *__restrict__ w = a.gamma;
  uint16_t *__restrict__ y = a.out;
  __shared__ float red[kPackedWaves];
  const int lane = threadIdx.x;
  const int nvec = a.cols >> 3;
  const size_t base = (size_t)blockIdx.x * a.cols;
  U4 pv[kPackedVpt];
  float ss = 0.f;
  bool ok = true;
#pragma unroll
  for (int i = 0; i < kPackedVpt; ++i) {
    const int c = lane + i * kPackedLanes;
    if (c < nvec) {
      U4 xw = ld16_once(x + base + (size_t)c * 8);
      float v[8];
      unpack8(xw, v);
      if constexpr (RESID) {
        float rv[8];
        unpack8(ld16_once(r + base + (size_t)c * 8), rv);
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = bf2f(f2bf(v[e] + rv[e]));
        xw = pack8(v);  // exact: the values are bf16
      }
      pv[i] = xw;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        ss += v[e] * v[e];
        ok &= div_elem_ok(v[e]);
      }
    }
  }
  ss = group_sum<kPackedWaves>(ss, red);
  const float rms = sqrtf(ss * a.inv_cols + a.eps);
  const bool fast = __all(ok && div_row_ok(rms));
  const float rinv = 1.0f / rms;
#pragma unroll
  for (int i = 0; i < kPackedVpt; ++i) {
    const int c = lane + i * kPackedLanes;
    if (c < nvec) {
      float v[8], o[8];
      unpack8(pv[i], v);
      if (fast) {
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = div_fast(v[e], rms, rinv);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = v[e] / rms;
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

template <int MODE>
__device__ __forceinline__ void softmax_packed_body(const RowArgs &a) {
#pragma clang fp contract(off)
  const void *__restrict__ in = a.in;
  const uint16_t *__restrict__ mask = a.aux;
  uint16_t *__restrict__ y = a.out;
  __shared__ float red[kPackedWaves];
  // chunks kPackedReg.. of every lane live in LDS: [chunk - kPackedReg][lane], 16 B each
  constexpr int kPackedReg = kPackedVpt / 2;
  __shared__ __attribute__((aligned(16))) U4 zl[kPackedVpt - kPackedReg][kPackedLanes];
  int lane = threadIdx.x;
  const int nvec = a.cols >> 3;
  const size_t base = (size_t)blockIdx.x * a.cols;
  U4 zp[kPackedReg];
  // Online sum while the row streams in: each lane keeps its running max ml and
  // sl = sum exp(z - ml), rescaled by exp(ml_old - ml) when ml grows, so the
  // exponentials of the sum overlap the loads and only the output pass
  // evaluates them again.  A lane that has seen only -inf keeps ml = -inf and
  // sl = 0.
  float ml = -INFINITY, sl = 0.f;
#pragma unroll
  for (int i = 0; i < kPackedVpt; ++i) {
    const int c = lane + i * kPackedLanes;
    if (c < nvec) {
      float z[8];
      load_z8<MODE>(in, mask, base + (size_t)c * 8, z);
      // (the index expression keeps the register array's index a constant in
      // both branches of the unrolled loop)
      if (i < kPackedReg) zp[i < kPackedReg ? i : 0] = pack8(z);  // exact: z are bf16 values
      else zl[i - kPackedReg][lane] = pack8(z);
      float cm = z[0];
#pragma unroll
      for (int e = 1; e < 8; ++e) cm = fmaxf(cm, z[e]);
      const float mn = fmaxf(ml, cm);
      if (mn != -INFINITY) {
        float t = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) t += expf(z[e] - mn);
        sl = sl * expf(ml - mn) + t;
        ml = mn;
      }
    }
  }
  const float m = group_max<kPackedWaves>(ml, red);
  auto chunk = [&](int i) __attribute__((always_inline)) -> U4 {
    return i < kPackedReg ? zp[i < kPackedReg ? i : 0] : zl[i - kPackedReg][lane];
  };
  // an opaque lane: the output pass recomputes its store addresses instead of
  // keeping 16 of them live across the reductions
  asm volatile("" : "+v"(lane));
  // a row of -inf only: m = -inf and every output is NaN, as exp(-inf - -inf)
  const float s = group_sum<kPackedWaves>(ml == -INFINITY ? 0.f : sl * expf(ml - m), red);
  const float inv = 1.0f / s;
#pragma unroll
  for (int i = 0; i < kPackedVpt; ++i) {
    const int c = lane + i * kPackedLanes;
    if (c < nvec) {
      float z[8], o[8];
      unpack8(chunk(i), z);
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = expf(z[e] - m) * inv;
      st16(y + base + (size_t)c * 8, pack8(o));
    }
  }
}

}  // namespace row
}  // namespace pk
