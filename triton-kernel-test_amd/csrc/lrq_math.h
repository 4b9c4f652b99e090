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
  return dy * (s * (1.f + x * (1.f - s)));
}

// gelu_backward.py:14-21 (tanh approximation): 0.5 * ((1 + t) + x * (1 - t^2) * g' ) * dy,
// t = tanh(gamma * (x + kappa * x^3)), g' = gamma * (1 + 3 * kappa * x^2).
__device__ __forceinline__ float gelu_bwd_f32(float x, float dy) {
  constexpr float kGamma = 0.7978845608028654f, kKappa = 0.044715f;
  const float x2 = x * x;
  const float u = kGamma * (x + kKappa * x2 * x);
  // tanh(u) = 1 - 2 / (exp(2u) + 1); saturates correctly at +-1.
  const float th = 1.f - 2.f * __builtin_amdgcn_rcpf(__expf(2.f * u) + 1.f);
  return 0.5f * ((1.f + th) + x * ((1.f - th * th) * kGamma * (1.f + 3.f * kKappa * x2))) * dy;
}

// fp32 -> nearest bf16 value, as fp32 (the rounding every bf16 torch op applies).
__device__ __forceinline__ float bf16r(float f) { return bf16_roundtrip(f); }

}  // namespace lrq
