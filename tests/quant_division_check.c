// The activation quantisation divides each value by its group scale s with one division per
// group (Markstein): y = RN(1/s), q = RN(x y), r = fma(-q, s, x), q' = copysign(RN(q + r y), x).
// This program checks, in binary32 with fused multiply-adds and no contraction, that q' equals
// x / s bit for bit wherever |x / s| >= 2^-12, and below that lies under e4m3's smallest step
// (2^-10) with x / s's sign, so the e4m3 codes agree everywhere. Inputs: 128-value groups of
// bf16 values (Gaussian, magnitudes 2^-40 .. 2^19, signed zeros) with s = amax / 448, and
// random (x, s) pairs with |x| <= 448 s; groups with s outside [2^-80, 2^100] are skipped (they
// divide).
// Usage: quant_division_check [groups]; exit status 1 on any mismatch.
#include <stdio.h>
#include <stdint.h>
#include <string.h>
#include <math.h>
#include <stdlib.h>
static float bf16_round(float f) { uint32_t u; memcpy(&u, &f, 4); u += 0x7fff + ((u >> 16) & 1); u &= 0xffff0000u; memcpy(&f, &u, 4); return f; }
static uint64_t st = 88172645463325252ull;
static uint64_t rnd(void) { st ^= st << 13; st ^= st >> 7; st ^= st << 17; return st; }
static double unif(void) { return (rnd() >> 11) * (1.0 / 9007199254740992.0); }
static double gauss(void) { double u = unif() + 1e-300, v = unif(); return sqrt(-2 * log(u)) * cos(6.283185307179586 * v); }
int main(int argc, char** argv) {
  long n = argc > 1 ? atol(argv[1]) : 10000000, bad = 0, checked = 0;
  for (long g = 0; g < n; ++g) {
    float x[128], amax = 0.f;
    const int e = (int)(rnd() % 60) - 40;                // group magnitudes 2^-40 .. 2^19
    for (int i = 0; i < 128; ++i) {
      float v = bf16_round((float)ldexp(gauss(), e));
      if (rnd() % 97 == 0) v = (rnd() & 1) ? 0.f : -0.f;
      x[i] = v; float a = fabsf(v); if (a > amax) amax = a;
    }
    float s = amax > 0.f ? amax / 448.0f : 1.0f;
    if (s < 0x1p-80f || s > 0x1p+100f) continue;
    float y = 1.0f / s;
    for (int i = 0; i < 128; ++i) {
      float q = x[i] * y;
      float r = fmaf(-q, s, x[i]);
      float q2 = copysignf(fmaf(r, y, q), x[i]);
      float ref = x[i] / s;
      uint32_t a, b; memcpy(&a, &q2, 4); memcpy(&b, &ref, 4);
      ++checked;
      const int mis = fabsf(ref) >= 0x1p-12f ? a != b : (!(fabsf(q2) < 0x1p-10f) || signbit(q2) != signbit(ref));
      if (mis) { if (bad < 5) printf("mismatch x=%a s=%a q2=%a ref=%a\n", x[i], s, q2, ref); ++bad; }
    }
  }
  // adversarial: x at many mantissas, s over a range of mantissas
  for (long i = 0; i < n; ++i) {
    uint32_t ub = 0x3f800000u | (uint32_t)(rnd() & 0x7fffff), ux = (uint32_t)(rnd() & 0xffff0000u);
    float s, xv; memcpy(&s, &ub, 4); memcpy(&xv, &ux, 4);
    s = ldexpf(s, (int)(rnd() % 100) - 60);
    if (!(fabsf(xv) <= 448.0f * s) || s < 0x1p-80f || s > 0x1p+100f) continue;
    float y = 1.0f / s, q = xv * y, r = fmaf(-q, s, xv), q2 = copysignf(fmaf(r, y, q), xv), ref = xv / s;
    uint32_t a, b; memcpy(&a, &q2, 4); memcpy(&b, &ref, 4); ++checked;
    const int mis = fabsf(ref) >= 0x1p-12f ? a != b : (!(fabsf(q2) < 0x1p-10f) || signbit(q2) != signbit(ref));
    if (mis) { if (bad < 10) printf("mismatch2 x=%a s=%a q2=%a ref=%a\n", xv, s, q2, ref); ++bad; }
  }
  printf("checked %ld values, %ld mismatches\n", checked, bad);
  return bad != 0;
}
