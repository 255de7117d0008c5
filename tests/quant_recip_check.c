// Exhaustive check of the fp32-scale e4m3 quant's reciprocal form
// (e4m3_quant4_recip in pih_amd/csrc/device_common.hpp): for every positive
// finite bf16 amax and every finite bf16 x with |x| <= amax, with
// s = RN(max(amax, 1e-4) / 448), r = RN(1 / s) and q0 = RN(x * r),
//   e4m3(clamp(RN(x / s))) == e4m3(clamp(copysign(fma(fma(-q0, s, x), r, q0), x)))
// where e4m3 is round-to-nearest-even onto e4m3fn codes.  Prints the pair
// count and the mismatches; exits 1 on any mismatch of a code.
#include <stdio.h>
#include <stdint.h>
#include <string.h>
#include <math.h>
#include <omp.h>
static float f(uint32_t u) { float x; memcpy(&x, &u, 4); return x; }
static uint32_t u(float x) { uint32_t v; memcpy(&v, &x, 4); return v; }
// e4m3fn RNE encode of |v| <= 448 finite
static uint32_t e4m3(float v) {
  uint32_t raw = u(v), sign = (raw >> 24) & 0x80, mag = raw & 0x7fffffff;
  if (mag == 0) return sign;
  int exp = (int)(mag >> 23) - 127;
  uint32_t code;
  if (exp < -6) code = (uint32_t)rintf(f(mag) * 512.0f);
  else {
    uint32_t mant = mag & 0x7fffff, q = mant >> 20, rem = mant & 0xfffff;
    if (rem > 0x80000 || (rem == 0x80000 && (q & 1))) ++q;
    int e = exp;
    if (q == 8) { q = 0; ++e; }
    code = ((uint32_t)(e + 7) << 3) | q;
  }
  return sign | code;
}
static float clampf(float v) { return fminf(fmaxf(v, -448.0f), 448.0f); }
int main(void) {
  long long bad = 0, total = 0, qdiff = 0;
  #pragma omp parallel for schedule(dynamic, 64) reduction(+:bad,total,qdiff)
  for (int ai = 0; ai <= 0x7f80; ++ai) {  // positive bf16 amax incl. +0 (floored) up to +inf exclusive
    if (ai == 0x7f80) continue;
    float amax = f((uint32_t)ai << 16);
    float s = fmaxf(amax, 1.0e-4f) / 448.0f;
    float r = 1.0f / s;
    for (uint32_t xi = 0; xi < 0x10000; ++xi) {
      float x = f(xi << 16);
      if (!isfinite(x) || fabsf(x) > amax) continue;
      float qd = x / s;
      float q0 = x * r;
      float res = fmaf(-q0, s, x);
      float q1 = copysignf(fmaf(res, r, q0), x);
      ++total;
      if (u(qd) != u(q1)) ++qdiff;
      if (e4m3(clampf(qd)) != e4m3(clampf(q1))) ++bad;
    }
  }
  printf("pairs %lld  fp32 quotient differs %lld  e4m3 code differs %lld\n", total, qdiff, bad);
  return bad != 0;
}
