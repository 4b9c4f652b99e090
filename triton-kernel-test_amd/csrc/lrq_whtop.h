// The 128-point Walsh-Hadamard rotation on one wave's 16 x 128 block (see lrq_wht.hip for the
// MFMA formulation), shared by the rotation kernels and the rotated decode.
#pragma once

#include "lrq_common.h"

namespace lrq {

// A operand of tile parity q0 for lane (i, kg): 8 bf16 signs for e = 0..7.
__device__ __forceinline__ u32x4 wht_base_operand(int i, int kg, int q0, bool neg) {
  const int v = i & 3, gp = i >> 2;
  uint32_t w[4];
#pragma unroll
  for (int h = 0; h < 4; ++h) {
    uint32_t pair = 0;
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const int e = 2 * h + s;
      const int par = (__builtin_popcount(v & e & 3) + (q0 & (e >> 2)) + __builtin_popcount(gp & kg) + (neg ? 1 : 0)) & 1;
      pair |= (par ? 0xbf80u : 0x3f80u) << (16 * s);
    }
    w[h] = pair;
  }
  return u32x4{w[0], w[1], w[2], w[3]};
}

// Rotate in place the 16 x 128 bf16 block whose lane (j, g) part (row j, columns 32g .. 32g+31)
// starts at `base` in LDS: y = bf16(fp32(sum_k H[o, k] x[k]) * fp32(1/sqrt(128))).
// op = the four wht_base_operand forms [q0][negated].
// f(k, y + 8k) gives the 8 bf16 stored for the lane's columns 32g + 8k .. +7 from their fp32
// rotated values (wht128_lds stores bf16(y); a fused consumer stores its result instead).
template <class F>
__device__ __forceinline__ void wht128_lds_map(unsigned char* base, const u32x4 (&op)[2][2], F f) {
  const float kScale = 0.08838834764831845f;  // fp32(1/sqrt(128))
  u32x4 xv[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) xv[c] = *reinterpret_cast<const u32x4*>(base + 16 * c);
  float out[32];
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    f32x4 acc = zero4();
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int flip = (((q >> 1) & c & 1) ^ ((q >> 2) & (c >> 1) & 1));
      acc = mfma_16x16x32(op[q & 1][flip], xv[c], acc);
    }
#pragma unroll
    for (int v = 0; v < 4; ++v) out[4 * q + v] = acc[v] * kScale;
  }
#pragma unroll
  for (int k = 0; k < 4; ++k) *reinterpret_cast<u32x4*>(base + 16 * k) = f(k, out + 8 * k);
}

__device__ __forceinline__ void wht128_lds(unsigned char* base, const u32x4 (&op)[2][2]) {
  wht128_lds_map(base, op, [](int, const float* y) { return pack8(y); });
}

}  // namespace lrq
