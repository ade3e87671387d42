// CPU check of the row kernels' division method (rowwise.hip div_fast)
// against IEEE x / d in round to nearest, for every bf16 numerator and n
// divisors (structured, the ends of the fast range, and random):
//   y = RN(1/d); q = RN(x y); e = fma(-q, d, x); result = fma(e, y, q)
// on the fast path (d in [2^-30, 2^30], |x| in [2^-64, 2^64]), x / d otherwise.
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
int main(int argc, char **argv) {
  long n = argc > 1 ? atol(argv[1]) : 2000;
  unsigned long long bad = 0, checked = 0, fastpath = 0;
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
