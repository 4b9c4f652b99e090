/* Exhaustive host check behind the legacy encode's division (csrc/lrq_legacy.hip,
 * legacy_code_rc): for every bf16 scale sc with 2^-100 <= |sc| <= 2^100 and every finite bf16
 * numerator a, the code clamp(rint(bf16(q)), -2^(b-1), 2^(b-1)-1) is the same for
 *   q = RN32(a / sc)                              (the reference's torch division), and
 *   q = fma(fma(-sc, q0, a), rc, q0),  q0 = med3(a * rc, -2^20, 2^20),  rc = RN32(1 / sc),
 * at b = 1, 2, 4 and 8.  Prints the number of pairs checked and of mismatches per bit width. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

static float bf(uint16_t h) { uint32_t u = (uint32_t)h << 16; float f; memcpy(&f, &u, 4); return f; }
static float bf16_round(float f) {  /* round to nearest even bf16 (finite or infinite input) */
  uint32_t u; memcpy(&u, &f, 4);
  u += 0x7fffu + ((u >> 16) & 1u);
  u &= 0xffff0000u;
  float r; memcpy(&r, &u, 4); return r;
}
static float med3(float x, float lo, float hi) { return x < lo ? lo : (x > hi ? hi : x); }
static int code(float q, int bits) {
  const float half = (float)(1 << (bits - 1));
  return (int)(med3(rintf(bf16_round(q)), -half, half - 1.f) + half);
}

int main(void) {
  long long checked = 0, bad1 = 0, bad2 = 0, bad4 = 0, bad8 = 0;
#pragma omp parallel for schedule(dynamic, 64) reduction(+ : checked, bad1, bad2, bad4, bad8)
  for (int s = 0; s < 65536; ++s) {
    const float sc = bf((uint16_t)s);
    const float m = fabsf(sc);
    if (!(m >= 0x1p-100f && m <= 0x1p100f)) continue;
    const float rc = 1.0f / sc;
    for (int h = 0; h < 65536; ++h) {
      const float a = bf((uint16_t)h);
      if (!isfinite(a)) continue;
      const float qr = a / sc;
      const float q0 = med3(a * rc, -0x1p20f, 0x1p20f);
      const float q = fmaf(fmaf(-sc, q0, a), rc, q0);
      ++checked;
      bad1 += code(qr, 1) != code(q, 1);
      bad2 += code(qr, 2) != code(q, 2);
      bad4 += code(qr, 4) != code(q, 4);
      bad8 += code(qr, 8) != code(q, 8);
    }
  }
  printf("%lld %lld %lld %lld %lld\n", checked, bad1, bad2, bad4, bad8);
  return 0;
}
