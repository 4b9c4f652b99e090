/* Exhaustive host check of the legacy MFMA encode's forms of the code step (csrc/lrq_legacy.hip):
 * for every fp32 quotient q that is not NaN (infinities included), the reference's code
 *   code(q, b) = clamp(rint(bf16(q)), -2^(b-1), 2^(b-1)-1) + 2^(b-1)
 * equals
 *   b = 1:        q >= -(0.5 + 2^-9)  (one compare, no rounding), and
 *   b = 2, 4, 8:  clamp(bits(d + 1.5 * 2^23), B - 2^(b-1), B + 2^(b-1) - 1) - B + 2^(b-1),
 *                 d = bf16(q), B = bits(1.5 * 2^23) (legacy_code_biased);
 *   b = 2 also:   [q > -(1.5 - 2^-8)] + [q >= -(0.5 + 2^-9)] + [q > 0.5 + 2^-9] (code2_thresholds);
 * and, at 1 and 2 bits, for every finite bf16 numerator a and bf16 scale sc with
 * 2^-100 <= |sc| <= 2^100 (the scales the reciprocal path serves), the compares of the
 * one-multiply estimate a * RN32(1/sc) give the codes of the IEEE quotient RN32(a / sc): no such
 * a / sc comes within 2^-17 of a threshold, far more than the estimate's error.
 * Prints the number of quotients checked and of mismatches per bit width (2 bits: both forms),
 * then the number of (a, sc) pairs checked and of mismatches of the 1- and 2-bit estimates. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

static float bf16_round(float f) { /* round to nearest even bf16 (finite or infinite input) */
  uint32_t u;
  memcpy(&u, &f, 4);
  u += 0x7fffu + ((u >> 16) & 1u);
  u &= 0xffff0000u;
  float r;
  memcpy(&r, &u, 4);
  return r;
}
static float med3(float x, float lo, float hi) { return x < lo ? lo : (x > hi ? hi : x); }
static int code(float q, int bits) {
  const float half = (float)(1 << (bits - 1));
  return (int)(med3(rintf(bf16_round(q)), -half, half - 1.f) + half);
}
static int code_biased(float q, int bits) {
  const int32_t bias = 0x4B400000, half = 1 << (bits - 1);
  volatile float s = bf16_round(q) + 0x1.8p23f; /* one fp32 add, rounded to nearest even */
  float sv = s;
  int32_t v;
  memcpy(&v, &sv, 4);
  v = v < bias - half ? bias - half : (v > bias + half - 1 ? bias + half - 1 : v);
  return v - bias + half;
}

static int code2_thresholds(float q) {
  return (q > -(1.5f - 0x1p-8f)) + (q >= -(0.5f + 0x1p-9f)) + (q > 0.5f + 0x1p-9f);
}

int main(void) {
  long long checked = 0, bad1 = 0, bad2 = 0, bad4 = 0, bad8 = 0;
#pragma omp parallel for schedule(dynamic, 1) reduction(+ : checked, bad1, bad2, bad4, bad8)
  for (int hi = 0; hi < 65536; ++hi) {
    for (int lo = 0; lo < 65536; ++lo) {
      const uint32_t u = ((uint32_t)hi << 16) | (uint32_t)lo;
      float q;
      memcpy(&q, &u, 4);
      if (isnan(q)) continue;
      ++checked;
      bad1 += code(q, 1) != (q >= -(0.5f + 0x1p-9f) ? 1 : 0);
      bad2 += (code(q, 2) != code_biased(q, 2)) + (code(q, 2) != code2_thresholds(q));
      bad4 += code(q, 4) != code_biased(q, 4);
      bad8 += code(q, 8) != code_biased(q, 8);
    }
  }
  long long pairs = 0, bad_est = 0, bad_est2 = 0;
#pragma omp parallel for schedule(dynamic, 64) reduction(+ : pairs, bad_est, bad_est2)
  for (int s = 0; s < 65536; ++s) {
    uint32_t us = (uint32_t)s << 16;
    float sc;
    memcpy(&sc, &us, 4);
    const float m = fabsf(sc);
    if (!(m >= 0x1p-100f && m <= 0x1p100f)) continue;
    const float rc = 1.0f / sc;
    for (int h = 0; h < 65536; ++h) {
      uint32_t ua = (uint32_t)h << 16;
      float a;
      memcpy(&a, &ua, 4);
      if (!isfinite(a)) continue;
      ++pairs;
      const float t = -(0.5f + 0x1p-9f);
      bad_est += (a * rc >= t) != (a / sc >= t);
      bad_est2 += code2_thresholds(a * rc) != code2_thresholds(a / sc);
    }
  }
  printf("%lld %lld %lld %lld %lld %lld %lld %lld\n", checked, bad1, bad2, bad4, bad8, pairs, bad_est, bad_est2);
  return 0;
}
