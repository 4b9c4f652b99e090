// Shared device helpers for the compressed-activation kernels (gfx950 / CDNA4, wave64).
//
// Lane conventions used by every kernel in this library.  A wave works on a block of
// 16 rows; lane l has j = l & 15 (row inside the block) and g = l >> 4 (0..3).  For a
// "chunk" of 32 consecutive columns starting at c0, lane (j, g) holds the 8 columns
// c0 + 8g .. c0 + 8g + 7 of row j as one 16-byte vector (4 dwords, two bf16 each,
// even column in the low half).  That is exactly the B operand of
// v_mfma_f32_16x16x32_bf16 with B = X^T, and — by choosing which V rows feed the A
// operand — the output layout of two v_mfma_f32_16x16x16_bf16 that compute L V^T for
// the same 32 columns.  So projection, residual and reconstruction never move
// activation data between lanes.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

namespace lrq {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

static constexpr int kWave = 64;

// ---------------------------------------------------------------- bf16 / fp16
__device__ __forceinline__ float bf_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// fp32 -> bf16 bits, round to nearest even (finite inputs; NaN becomes a quiet NaN).
__device__ __forceinline__ uint32_t bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0u;
  u += 0x7fffu + ((u >> 16) & 1u);
  return u >> 16;
}
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return bf16_bits(lo) | (bf16_bits(hi) << 16);
}
__device__ __forceinline__ float bf16_roundtrip(float f) { return __uint_as_float(bf16_bits(f) << 16); }

// fp32 -> fp16 bits (RNE) and back.
__device__ __forceinline__ uint16_t f16_bits(float f) {
  return __builtin_bit_cast(uint16_t, (_Float16)f);
}
__device__ __forceinline__ float f16_val(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }

// ---------------------------------------------------------------- MFMA wrappers
// D(16x16) += A(16x32) * B(32x16), bf16 inputs, fp32 accumulate.
__device__ __forceinline__ f32x4 mfma_16x16x32(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                 __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}
// D(16x16) += A(16x16) * B(16x16), bf16 inputs, fp32 accumulate.
__device__ __forceinline__ f32x4 mfma_16x16x16(u32x2 a, u32x2 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s16x4, a),
                                                   __builtin_bit_cast(s16x4, b), c, 0, 0, 0);
}

// ---------------------------------------------------------------- memory helpers
__device__ __forceinline__ u32x4 ld16(const void* p) { return *reinterpret_cast<const u32x4*>(p); }
__device__ __forceinline__ u32x2 ld8(const void* p) { return *reinterpret_cast<const u32x2*>(p); }
__device__ __forceinline__ u32x4 ld16_stream(const void* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}
__device__ __forceinline__ u32x2 ld8_stream(const void* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(p));
}
__device__ __forceinline__ void st16(void* p, u32x4 v) { *reinterpret_cast<u32x4*>(p) = v; }
__device__ __forceinline__ void st8(void* p, u32x2 v) { *reinterpret_cast<u32x2*>(p) = v; }
__device__ __forceinline__ void st16_stream(void* p, u32x4 v) {
  __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(p));
}

// Unpack the 8 bf16 of a 16-byte vector into fp32.
__device__ __forceinline__ void unpack8(u32x4 v, float* f) {
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    f[2 * d] = bf_lo(v[d]);
    f[2 * d + 1] = bf_hi(v[d]);
  }
}
__device__ __forceinline__ u32x4 pack8(const float* f) {
  u32x4 v;
#pragma unroll
  for (int d = 0; d < 4; ++d) v[d] = pack_bf16x2(f[2 * d], f[2 * d + 1]);
  return v;
}

// ---------------------------------------------------------------- low-rank reconstruction
// P[j][c0 + 8g + e], e = 0..7, for the lane's row j, using the residual-operand trick:
// MFMA h (h = 0, 1) feeds A row i = j with V row c0 + 8*(i/4) + 4h + (i%4), so its output
// lands in lane (j, g) as columns c0 + 8g + 4h + v.  `lop[t]` is the B operand of rank
// tile t: L[j][16t + 4g .. 16t + 4g + 3] as 4 packed bf16.  V is [N][R] bf16, row-major.
template <int R>
__device__ __forceinline__ void lowrank_chunk(const uint16_t* __restrict__ V, int c0, int j, int g,
                                              const u32x2* lop, float* p) {
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int vrow = c0 + 8 * (j >> 2) + 4 * h + (j & 3);
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int t = 0; t < R / 16; ++t) {
      u32x2 a = ld8(V + (int64_t)vrow * R + 16 * t + 4 * g);
      acc = mfma_16x16x16(a, lop[t], acc);
    }
    p[4 * h + 0] = acc[0];
    p[4 * h + 1] = acc[1];
    p[4 * h + 2] = acc[2];
    p[4 * h + 3] = acc[3];
  }
}

// Cross-lane reductions over the 4 lanes that share a row (lanes j, j+16, j+32, j+48).
__device__ __forceinline__ float wave_min4(float v) {
  v = fminf(v, __shfl_xor(v, 16));
  v = fminf(v, __shfl_xor(v, 32));
  return v;
}
__device__ __forceinline__ float wave_max4(float v) {
  v = fmaxf(v, __shfl_xor(v, 16));
  v = fmaxf(v, __shfl_xor(v, 32));
  return v;
}
__device__ __forceinline__ float wave_sum4(float v) {
  v += __shfl_xor(v, 16);
  v += __shfl_xor(v, 32);
  return v;
}

// ---------------------------------------------------------------- group quantiser
// Per-group parameters from min/max, exactly as the CPU oracle defines them:
//   scale_h = fp16(min((mx - mn) / qmax, 65504)), 1 when that is 0; zero_h = fp16(clamp(mn));
//   inv = 1 / fp32(scale_h).  Division is IEEE correctly rounded (HIP default).
struct GroupParams {
  float inv, zf;
  uint16_t sh, zh;
};
template <int BITS>
__device__ __forceinline__ GroupParams group_params(float mn, float mx) {
  constexpr float qmax = (float)((1 << BITS) - 1);
  GroupParams gp;
  float s = (mx - mn) / qmax;
  s = fminf(s, 65504.f);
  uint16_t sh = f16_bits(s);
  if ((sh & 0x7fffu) == 0) sh = 0x3c00u;  // 1.0
  float z = fminf(fmaxf(mn, -65504.f), 65504.f);
  gp.sh = sh;
  gp.zh = f16_bits(z);
  gp.zf = f16_val(gp.zh);
  gp.inv = 1.0f / f16_val(sh);
  return gp;
}
// code = clamp(rint((r - zf) * inv), 0, qmax); the subtract and the multiply round separately.
template <int BITS>
__device__ __forceinline__ uint32_t quant_code(float r, const GroupParams& gp) {
  constexpr float qmax = (float)((1 << BITS) - 1);
  float t = __fmul_rn(__fsub_rn(r, gp.zf), gp.inv);
  t = __builtin_rintf(t);
  t = fminf(fmaxf(t, 0.f), qmax);
  return (uint32_t)t;
}

}  // namespace lrq
