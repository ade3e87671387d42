// CPU check of the row kernels' division method (rowwise.hip div_fast)
// against IEEE x / d in round to nearest, for every bf16 numerator and n
// divisors (structured, the ends of the fast range, and random):
//   y = RN(1/d); q = RN(x y); e = fma(-q, d, x); result = fma(e, y, q)
// on the fast path (d in [2^-30, 2^30], |x| in [2^-64, 2^64]), x / d otherwise.
// Also checks the packed range test that selects the fast path (check_span).
// Build with -ffp-contract=off so every multiply and add rounds separately.
// Exit status 0 when no result differs.
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
static float bf(uint16_t b) { uint32_t u = (uint32_t)b << 16; float f; memcpy(&f, &u, 4); return f; }
static uint32_t bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
// fast path when d in [2^-30, 2^30] and |x| in [2^-64, 2^64]
static float fastdiv(float x, float d, float y) {
  float ax = fabsf(x);
  if (!(ax >= 0x1p-64f && ax <= 0x1p64f)) return x / d;
  float q = x * y;
#ifdef PK_PLANT_NO_CORRECTION
  return q;  /* a deliberately wrong method: the check must catch it */
#else
  float e = fmaf(-q, d, x);
  return fmaf(e, y, q);
#endif
}
// The kernels' packed range test (pk_common.hpp DivSpan): a 32-bit word of
// two bf16 numerators qualifies when both magnitudes (bits & 0x7FFF) lie in
// [0x1F80, 0x5F80).  It must accept exactly the words whose two values satisfy
// 2^-64 <= |x| < 2^64 (the float test).
static int span_ok(uint32_t w) {
  const uint32_t lo = w & 0x7FFFu, hi = (w >> 16) & 0x7FFFu;
  const uint32_t mn = lo < hi ? lo : hi, mx = lo > hi ? lo : hi;
#ifdef PK_PLANT_SPAN_BOUND
  return mn >= 0x1F80u && mx <= 0x5F80u;  /* a deliberately wrong bound: 2^64 accepted */
#else
  return mn >= 0x1F80u && mx < 0x5F80u;
#endif
}
static int float_ok(uint16_t b) {
  const float a = fabsf(bf(b));
  return a >= 0x1p-64f && a < 0x1p64f;
}
static unsigned long long check_span(void) {
  unsigned long long bad = 0;
  for (uint32_t b = 0; b < 65536; ++b)
    for (uint32_t k = 0; k < 65536; k += 251) {  // every code against 262 partners, both orders
      const uint32_t c = (b * 40503u + k) & 0xFFFFu;
      const int want = float_ok((uint16_t)b) && float_ok((uint16_t)c);
      if (span_ok(b | (c << 16)) != want || span_ok(c | (b << 16)) != want) {
        if (bad < 5) printf("span mismatch %04x %04x\n", b, c);
        ++bad;
      }
    }
  for (uint32_t b = 0; b < 65536; ++b)  // every code with itself and with 1.0
    if (span_ok(b | (b << 16)) != float_ok((uint16_t)b) || span_ok(b | (0x3F80u << 16)) != float_ok((uint16_t)b))
      ++bad;
  return bad;
}
int main(int argc, char **argv) {
  long n = argc > 1 ? atol(argv[1]) : 2000;
  unsigned long long bad = 0, checked = 0, fastpath = 0;
  const unsigned long long span_bad = check_span();
  printf("span mismatches %llu\n", span_bad);
  bad += span_bad;
  srand(12345);
  for (long i = 0; i < n; ++i) {
    float d;
    if (i < 64) {  // structured: 1, powers of two, rms-like values near sqrt(eps)
      d = ldexpf(1.0f + (float)i / 64.0f, (int)(i % 13) - 6);
    } else if (i < 96) {  // the ends of the fast range, all-ones and minimal mantissas
      const int j = (int)i - 64;
      d = ldexpf((j & 1) ? 1.99999988f : 1.0f, (j & 2) ? 29 : -30) * ((j & 4) ? 1.0f : 1.00000012f);
    } else {
      // rms = sqrt(ss/cols + eps) over plausible ranges, random mantissas
      uint32_t u = ((uint32_t)rand() << 16) ^ (uint32_t)rand();
      int ex = 127 + (rand() % 61) - 30;  // 2^-30 .. 2^30
      u = (u & 0x7FFFFFu) | ((uint32_t)ex << 23);
      memcpy(&d, &u, 4);
    }
    float y = 1.0f / d;
    int dok = isfinite(d) && fabsf(d) >= 0x1p-30f && fabsf(d) <= 0x1p30f;
    for (uint32_t b = 0; b < 65536; ++b) {
      float x = bf((uint16_t)b);
      float ref = x / d;
      float got = dok ? fastdiv(x, d, y) : x / d;
      ++checked;
      if (dok) fastpath += (fabsf(x) >= 0x1p-64f && fabsf(x) <= 0x1p64f);
      if (isnan(ref) ? !isnan(got) : bits(ref) != bits(got)) {
        if (bad < 5) printf("mismatch x=%a d=%a ref=%a got=%a\n", x, d, ref, got);
        ++bad;
      }
    }
  }
  printf("checked %llu, fast path %llu, mismatches %llu\n", checked, fastpath, bad);
  return bad != 0;
}
