// The 128-point Walsh-Hadamard rotation on one wave's 16 x 128 block (see lrq_wht.hip for the
// MFMA formulation), shared by the rotation kernels and the rotated decode.
#pragma once

#include "lrq_common.h"

namespace lrq {

// Dword h (bf16 signs of e = 2h, 2h+1) of the A operand of tile parity q0 for lane (i, kg):
// the sign of element e is (-1)^(popcount(i & e & 3) + (q0 & (e >> 2)) + popcount((i >> 2) & kg) + neg).
__host__ __device__ constexpr uint32_t wht_sign_dword(int i, int kg, int q0, bool neg, int h) {
  uint32_t pair = 0;
  for (int s = 0; s < 2; ++s) {
    const int e = 2 * h + s;
    const int par = (__builtin_popcount((unsigned)(i & 3 & e & 3)) + (q0 & (e >> 2)) +
                     __builtin_popcount((unsigned)((i >> 2) & kg)) + (neg ? 1 : 0)) & 1;
    pair |= (par ? 0xbf80u : 0x3f80u) << (16 * s);
  }
  return pair;
}

// Every operand of a lane is built from its two dwords A = dword 0 and B = dword 1 of the
// (q0 = 0, neg = false) form: (A, B, A, B) for q0 = 0 and (A, B, A^F, B^F) for q0 = 1, all xor F
// when negated (F = 0x80008000 flips both bf16 signs).  Checked for every lane and form:
constexpr bool wht_sign_pair_form_holds() {
  constexpr uint32_t F = 0x80008000u;
  for (int i = 0; i < 16; ++i)
    for (int kg = 0; kg < 4; ++kg)
      for (int q0 = 0; q0 < 2; ++q0)
        for (int n = 0; n < 2; ++n) {
          const uint32_t a = wht_sign_dword(i, kg, 0, false, 0), b = wht_sign_dword(i, kg, 0, false, 1);
          const uint32_t want[4] = {a, b, q0 ? a ^ F : a, q0 ? b ^ F : b};
          for (int h = 0; h < 4; ++h)
            if (wht_sign_dword(i, kg, q0, n != 0, h) != (n ? want[h] ^ F : want[h])) return false;
        }
  return true;
}
static_assert(wht_sign_pair_form_holds(), "WHT sign operands from two dwords per lane");

// The four operand forms [q0][negated] of a lane from its two dwords (see above).
__device__ __forceinline__ void wht_operands_from_pair(uint32_t a, uint32_t b, u32x4 (&op)[2][2]) {
  constexpr uint32_t F = 0x80008000u;
  op[0][0] = u32x4{a, b, a, b};
  op[0][1] = u32x4{a ^ F, b ^ F, a ^ F, b ^ F};
  op[1][0] = u32x4{a, b, a ^ F, b ^ F};
  op[1][1] = u32x4{a ^ F, b ^ F, a, b};
}

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
// at(c) is the LDS address of the lane's 16-byte chunk c (columns 32g + 8c .. +7).
template <class A, class F>
__device__ __forceinline__ void wht128_lds_at(A at, const u32x4 (&op)[2][2], F f) {
  const float kScale = 0.08838834764831845f;  // fp32(1/sqrt(128))
  u32x4 xv[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) xv[c] = *reinterpret_cast<const u32x4*>(at(c));
  // two halves of the outputs (chunks 0-1, then 2-3): every input is in registers already,
  // and half the output registers are live at a time
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    float out[16];
#pragma unroll
    for (int qq = 0; qq < 4; ++qq) {
      const int q = 4 * h + qq;
      f32x4 acc = zero4();
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int flip = (((q >> 1) & c & 1) ^ ((q >> 2) & (c >> 1) & 1));
        acc = mfma_16x16x32(op[q & 1][flip], xv[c], acc);
      }
#pragma unroll
      for (int v = 0; v < 4; ++v) out[4 * qq + v] = acc[v] * kScale;
    }
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) *reinterpret_cast<u32x4*>(at(2 * h + kk)) = f(2 * h + kk, out + 8 * kk);
  }
}

template <class F>
__device__ __forceinline__ void wht128_lds_map(unsigned char* base, const u32x4 (&op)[2][2], F f) {
  wht128_lds_at([base](int c) { return base + 16 * c; }, op, f);
}

__device__ __forceinline__ void wht128_lds(unsigned char* base, const u32x4 (&op)[2][2]) {
  wht128_lds_map(base, op, [](int, const float* y) { return pack8(y); });
}

// The rotation of one 16 x 128 block held in registers, for kernels whose lanes rebuild a
// block's columns themselves.  The decode's wht128_lds gives lane group g the block's columns
// 32g .. 32g+31 (chunk c = columns 32g + 8c .. +7, so MFMA step c sums the 32 columns
// {32g' + 8c + e}); a lane of the G/4-column reconstruction layout holds columns E g .. of each
// of the block's 128/G units instead.  rot_gather_128 packs the lane's 32 values of row j to bf16
// in the order of wht128_lds: for G = 128 they already are columns 32g + i; for G = 64 one
// v_permlane16_swap per dword pair of the two units' quarters gives lane group g the columns
// 32 sigma(g) .. +31, sigma(g) = (0, 2, 1, 3)[g], and the lane's sign operands are built for
// group sigma(g) (rot_sign_group).  Each MFMA step then sums the same 32 products as the
// decode's, so the rotated values are the decode's bit for bit.
template <int G>
__device__ __forceinline__ int rot_sign_group(int g) {
  static_assert(G == 64 || G == 128, "64- or 128-column units");
  return G == 128 ? g : ((g & 1) << 1) | (g >> 1);
}
template <int G>
__device__ __forceinline__ void rot_gather_128(const float* xh, u32x4 (&xv)[4]) {
#pragma unroll
  for (int c = 0; c < 4; ++c) xv[c] = pack8(xh + 8 * c);  // bf16(Y')
  if constexpr (G == 64) {
    // xv[0..1]: unit 0, columns 16g .. +15; xv[2..3]: unit 1, columns 64 + 16g .. +15
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        const auto s = __builtin_amdgcn_permlane16_swap(xv[c][d], xv[c + 2][d], false, false);
        xv[c][d] = s[0];
        xv[c + 2][d] = s[1];
      }
  }
}
// Rotate the gathered block: y[s] = fp32(sum) * fp32(1/sqrt(128)) of row j, column 32g + s of the
// block (s < 32), before the bf16 rounding; op = the four wht_base_operand forms of
// (j, rot_sign_group<G>(g)).
__device__ __forceinline__ void wht128_regs(const u32x4 (&xv)[4], const u32x4 (&op)[2][2], float* y) {
  const float kScale = 0.08838834764831845f;  // fp32(1/sqrt(128)), as in wht128_lds_at
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    f32x4 acc = zero4();
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int flip = (((q >> 1) & c & 1) ^ ((q >> 2) & (c >> 1) & 1));
      acc = mfma_16x16x32(op[q & 1][flip], xv[c], acc);
    }
#pragma unroll
    for (int v = 0; v < 4; ++v) y[4 * q + v] = acc[v] * kScale;
  }
}

// wht128_lds on a row of a swizzled tile: the row's 16-byte chunk c (columns 8c .. 8c+7 of the
// 128) sits at row + 16 * (c ^ sw), sw < 16; the lane's chunks are 4g .. 4g+3.
__device__ __forceinline__ void wht128_lds_swz(unsigned char* row, int g, int sw, const u32x4 (&op)[2][2]) {
  wht128_lds_at([=](int c) { return row + 16 * ((4 * g + c) ^ sw); }, op,
                [](int, const float* y) { return pack8(y); });
}

}  // namespace lrq
