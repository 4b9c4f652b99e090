/* Exhaustive host check of the legacy MFMA encode's code step (csrc/lrq_legacy.hip).  The
 * reference's code of a quotient q (low_rank_extraction_fuse_compression_quantization.py:165-166,
 * torch form) is
 *   code(q, b) = clamp(rint(bf16(q)), -2^(b-1), 2^(b-1)-1) + 2^(b-1),   q = RN32(a / sc),
 * with a = x - l r - o and sc bf16 values.  The encode takes
 *   1. for every fp32 q that is not NaN (infinities included):
 *        b = 1:        q >= -(0.5 + 2^-9)  (one compare, no rounding), and
 *        b = 2, 4, 8:  clamp(bits(d + 1.5 * 2^23), B - 2^(b-1), B + 2^(b-1) - 1) - B + 2^(b-1),
 *                      d = bf16(q), B = bits(1.5 * 2^23) (legacy_code_biased);
 *   2. for every finite bf16 a and bf16 sc with 2^-100 <= |sc| <= 2^100 (the scales the
 *      estimate serves) the quotient estimate a * RN32(1/sc) in place of RN32(a / sc): its code is
 *      the same at b = 1, 2, 4 and 8 (a / sc never comes near a code boundary within the
 *      estimate's error).
 * Prints the number of quotients checked and of mismatches of part 1 per bit width, then the
 * number of (a, sc) pairs checked and of mismatches of part 2 per bit width. */
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
static float from_bits(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}

int main(void) {
  long long checked = 0, bad1 = 0, bad2 = 0, bad4 = 0, bad8 = 0;
#pragma omp parallel for schedule(dynamic, 1) reduction(+ : checked, bad1, bad2, bad4, bad8)
  for (int hi = 0; hi < 65536; ++hi) {
    for (int lo = 0; lo < 65536; ++lo) {
      const float q = from_bits(((uint32_t)hi << 16) | (uint32_t)lo);
      if (isnan(q)) continue;
      ++checked;
      bad1 += code(q, 1) != (q >= -(0.5f + 0x1p-9f) ? 1 : 0);
      bad2 += code(q, 2) != code_biased(q, 2);
      bad4 += code(q, 4) != code_biased(q, 4);
      bad8 += code(q, 8) != code_biased(q, 8);
    }
  }
  long long pairs = 0, e1 = 0, e2 = 0, e4 = 0, e8 = 0;
#pragma omp parallel for schedule(dynamic, 64) reduction(+ : pairs, e1, e2, e4, e8)
  for (int s = 0; s < 65536; ++s) {
    const float sc = from_bits((uint32_t)s << 16);
    const float m = fabsf(sc);
    if (!(m >= 0x1p-100f && m <= 0x1p100f)) continue;
    const float rc = 1.0f / sc;
    for (int h = 0; h < 65536; ++h) {
      const float a = from_bits((uint32_t)h << 16);
      if (!isfinite(a)) continue;
      ++pairs;
      const float est = a * rc, q = a / sc;
      e1 += code(est, 1) != code(q, 1);
      e2 += code(est, 2) != code(q, 2);
      e4 += code(est, 4) != code(q, 4);
      e8 += code(est, 8) != code(q, 8);
    }
  }
  printf("%lld %lld %lld %lld %lld %lld %lld %lld %lld %lld\n", checked, bad1, bad2, bad4, bad8, pairs, e1, e2, e4,
         e8);
  return 0;
}
