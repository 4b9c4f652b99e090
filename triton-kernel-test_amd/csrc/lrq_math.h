// Elementwise consumer math shared by the fused decode epilogues, the legacy kernels and the
// dense kernels.  All fp32, one bf16 rounding at the end (done by the caller), as
// torch.ops.aten.silu_backward / gelu_backward(approximate='tanh') compute it.
#pragma once

#include "lrq_common.h"

namespace lrq {

// silu_backward.py:6-8 / extraction_fuse_silu_backward.py:10-13:
// dy * s * (1 + x * (1 - s)), s = sigmoid(x).
__device__ __forceinline__ float silu_bwd_f32(float x, float dy) {
  const float s = __builtin_amdgcn_rcpf(1.f + __expf(-x));
  return dy * (s * __builtin_fmaf(x, 1.f - s, 1.f));
}

// gelu_backward.py:14-21 (tanh approximation): 0.5 * ((1 + t) + x * (1 - t^2) * g' ) * dy,
// t = tanh(gamma * (x + kappa * x^3)), g' = gamma * (1 + 3 * kappa * x^2).
// With s = sigmoid(2u) (u the tanh argument): 1 + t = 2s and 1 - t^2 = 4s(1 - s), so the
// derivative is s * (1 + 2x g' (1 - s)): one exp, one reciprocal and 11 other operations.
__device__ __forceinline__ float gelu_bwd_f32(float x, float dy) {
  constexpr float kGamma = 0.7978845608028654f, kKappa = 0.044715f;
  constexpr float kLog2e = 1.4426950408889634f;
  const float x2 = x * x;
  const float u2 = x * __builtin_fmaf(2.f * kGamma * kKappa, x2, 2.f * kGamma);  // 2u
  const float s = __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(-kLog2e * u2));
  const float g2 = x * __builtin_fmaf(6.f * kGamma * kKappa, x2, 2.f * kGamma);  // 2x g'
  return (s * __builtin_fmaf(g2, 1.f - s, 1.f)) * dy;
}

// fp32 -> nearest bf16 value, as fp32 (the rounding every bf16 torch op applies).
__device__ __forceinline__ float bf16r(float f) { return bf16_roundtrip(f); }

}  // namespace lrq
