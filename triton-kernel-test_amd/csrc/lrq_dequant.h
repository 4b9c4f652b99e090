// Dequantisation + low-rank reconstruction of one unit-plane (see lrq_common.h for the
// layout), shared by the decode, the fused consumers, the softmax backward and the
// dequant-GEMM kernels.
#pragma once

#include "lrq_common.h"

namespace lrq {

// xh[e] = fp32(code_e * scale + zero + (L V^T)[row, col_e]) for the lane's G/4 columns of
// plane p: cb holds the lane's G/4 code bytes of the unit (plane p in bits BITS*p ..),
// qp the plane's (scale, zero) fp16 pair.  code * scale is exact, so the fma rounds once,
// like the oracle's multiply-add, and the low-rank term is added inside the MFMA
// accumulation (one more rounding).
template <int BITS, int G, int R>
__device__ __forceinline__ void reconstruct_plane(const u32x4 (&cb)[G / 64], uint32_t qp, int p,
                                                  const u32x2 (&vop)[G / 16][R > 0 ? R / 16 : 1],
                                                  const u32x2* lop, float* xh) {
  constexpr int NP = 8 / BITS, E = G / 4;
  constexpr uint32_t kMask = (1u << BITS) - 1u;
  const float sf = f16_val(qp & 0xffffu);
  const float zf = f16_val(qp >> 16);
#pragma unroll
  for (int d = 0; d < E / 4; ++d) {
    // the codes of plane p for elements 4d .. 4d+3, one per byte
    const uint32_t wd = cb[d >> 2][d & 3];
    const uint32_t wq = NP == 1 ? wd : ((wd >> (BITS * p)) & (0x01010101u * kMask));
    xh[4 * d + 0] = __builtin_fmaf(ubyte_f32<0>(wq), sf, zf);
    xh[4 * d + 1] = __builtin_fmaf(ubyte_f32<1>(wq), sf, zf);
    xh[4 * d + 2] = __builtin_fmaf(ubyte_f32<2>(wq), sf, zf);
    xh[4 * d + 3] = __builtin_fmaf(ubyte_f32<3>(wq), sf, zf);
  }
  if constexpr (R > 0) residual_unit<G, R>(vop, lop, xh, xh);
}

}  // namespace lrq
