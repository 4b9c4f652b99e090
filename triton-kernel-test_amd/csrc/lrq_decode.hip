// Group-mode decode and the fused elementwise consumers (SiLU backward, GELU backward,
// elementwise product).  One streaming pass: codes, scales and L are read once, the
// low-rank term L V^T is rebuilt on MFMA in the lanes that own the columns, and the
// epilogue either stores x_hat (bf16, non-temporal) or applies the consumer with the
// upstream gradient so the full-precision activation never goes back to HBM.
#include "lrq_common.h"
#include "lrq_host.h"

namespace lrq {

// ------------------------------------------------------------------ epilogues
// Each receives 8 consecutive reconstructed values (fp32, before the bf16 rounding that
// defines x_hat) for row `row`, columns col .. col + 7.
struct EpiStore {
  uint16_t* out;
  int64_t ld;
  __device__ __forceinline__ void operator()(int64_t row, int col, const float* xh, bool rv) const {
    if (rv) st16_stream(out + row * ld + col, pack8(xh));
  }
};

// silu_backward.py:6-8: dy * (s * (1 + x * (1 - s))), s = sigmoid(x), x = bf16(x_hat); fp32.
struct EpiSilu {
  const uint16_t* dy;
  int64_t lddy;
  uint16_t* dx;
  int64_t lddx;
  __device__ __forceinline__ void operator()(int64_t row, int col, const float* xh, bool rv) const {
    if (!rv) return;
    float d[8], o[8];
    unpack8(ld16_stream(dy + row * lddy + col), d);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float x = bf16_roundtrip(xh[e]);
      const float s = __builtin_amdgcn_rcpf(1.f + __expf(-x));
      o[e] = d[e] * (s * (1.f + x * (1.f - s)));
    }
    st16_stream(dx + row * lddx + col, pack8(o));
  }
};

// gelu_backward.py:14-21 (tanh approximation), fp32 on x = bf16(x_hat).
struct EpiGelu {
  const uint16_t* dy;
  int64_t lddy;
  uint16_t* dx;
  int64_t lddx;
  __device__ __forceinline__ void operator()(int64_t row, int col, const float* xh, bool rv) const {
    if (!rv) return;
    constexpr float kGamma = 0.7978845608028654f, kKappa = 0.044715f;
    float d[8], o[8];
    unpack8(ld16_stream(dy + row * lddy + col), d);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float x = bf16_roundtrip(xh[e]);
      const float x2 = x * x;
      const float u = kGamma * (x + kKappa * x2 * x);
      // tanh(u) = 1 - 2 / (exp(2u) + 1); saturates correctly at +-1.
      const float th = 1.f - 2.f * __builtin_amdgcn_rcpf(__expf(2.f * u) + 1.f);
      o[e] = 0.5f * ((1.f + th) + x * ((1.f - th * th) * kGamma * (1.f + 3.f * kKappa * x2))) * d[e];
    }
    st16_stream(dx + row * lddx + col, pack8(o));
  }
};

// extraction_fuse_hadamard.py:5-6: x * y.
struct EpiMul {
  const uint16_t* y;
  int64_t ldy;
  uint16_t* out;
  int64_t ldo;
  __device__ __forceinline__ void operator()(int64_t row, int col, const float* xh, bool rv) const {
    if (!rv) return;
    float a[8], o[8];
    unpack8(ld16_stream(y + row * ldy + col), a);
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = bf16_roundtrip(xh[e]) * a[e];
    st16_stream(out + row * ldo + col, pack8(o));
  }
};

// ------------------------------------------------------------------ kernel
// Grid: (ceil(rows / 64), ceil(units / upb)), 256 threads = 4 waves x 16 rows.  A unit is
// CPG = G/32 consecutive chunks of every packing plane (see lrq_quant.h); the 8 bytes lane
// (j, g) reads for chunk k hold the codes of columns c0 + 8g + e of all NP planes.
template <int BITS, int G, int R, bool OUTL, class EPI>
__global__ __launch_bounds__(256) void k_decode(
    const uint8_t* __restrict__ codes, int64_t ldc, const uint16_t* __restrict__ scale,
    const uint16_t* __restrict__ zero, int64_t ldsz, const uint16_t* __restrict__ Lin, int64_t ldl,
    const uint16_t* __restrict__ V, int M, int N, const int32_t* __restrict__ oidx, int nout,
    const uint16_t* __restrict__ side, int64_t ldside, int upb, EPI epi) {
  constexpr int NP = 8 / BITS, CPG = G / 32, RT = R > 0 ? R / 16 : 1;
  constexpr uint32_t kMask = (1u << BITS) - 1u;
  extern __shared__ uint32_t smem[];
  uint32_t* colmask = smem;                               // N/32 words
  int16_t* slot = reinterpret_cast<int16_t*>(smem + N / 32);  // N entries
  const int PC = N / (32 * NP);
  const int units = PC / CPG;
  if constexpr (OUTL) {
    for (int i = threadIdx.x; i < N / 32; i += blockDim.x) colmask[i] = 0u;
    for (int i = threadIdx.x; i < N; i += blockDim.x) slot[i] = -1;
    __syncthreads();
    for (int k = threadIdx.x; k < nout; k += blockDim.x) {
      const int c = oidx[k];
      if (c >= 0 && c < N) {
        atomicOr(&colmask[c >> 5], 1u << (c & 31));
        slot[c] = (int16_t)k;
      }
    }
    __syncthreads();
  }
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int j = lane & 15, g = lane >> 4;
  const int row = blockIdx.x * 64 + w * 16 + j;
  const bool rv = row < M;
  const int64_t rr = rv ? row : 0;
  u32x2 lop[RT];
  if constexpr (R > 0) {
#pragma unroll
    for (int t = 0; t < RT; ++t) lop[t] = rv ? ld8(Lin + rr * ldl + 16 * t + 4 * g) : u32x2{0u, 0u};
  }
  const uint8_t* crow = codes + rr * ldc;
  for (int ui = 0; ui < upb; ++ui) {
    const int u = blockIdx.y * upb + ui;
    if (u >= units) break;
    const int cu = u * CPG;
    u32x2 cb[CPG];
#pragma unroll
    for (int k = 0; k < CPG; ++k) cb[k] = rv ? ld8_stream(crow + (cu + k) * 32 + 8 * g) : u32x2{0u, 0u};
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      const int gi = ((p * PC + cu) * 32) / G;
      const float sf = f16_val(scale[rr * ldsz + gi]);
      const float zf = f16_val(zero[rr * ldsz + gi]);
#pragma unroll
      for (int k = 0; k < CPG; ++k) {
        const int c0 = (p * PC + cu + k) * 32;
        float xh[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const uint32_t code = (cb[k][e >> 2] >> (8 * (e & 3) + BITS * p)) & kMask;
          xh[e] = __builtin_fmaf((float)code, sf, zf);  // code * scale is exact
        }
        if constexpr (R > 0) {
          float pl[8];
          lowrank_chunk<R>(V, c0, j, g, lop, pl);
#pragma unroll
          for (int e = 0; e < 8; ++e) xh[e] = __fadd_rn(xh[e], pl[e]);
        }
        if constexpr (OUTL) {
          const uint32_t mbits = (colmask[c0 >> 5] >> (8 * g)) & 0xffu;
          if (mbits && rv) {
#pragma unroll
            for (int e = 0; e < 8; ++e)
              if ((mbits >> e) & 1u) xh[e] = f16_val(side[rr * ldside + slot[c0 + 8 * g + e]]);
          }
        }
        epi(rr, c0 + 8 * g, xh, rv);
      }
    }
  }
}

// ------------------------------------------------------------------ host side
template <int BITS, int G, int R, class EPI>
static int decode_launch(const lrq_tensors* t, hipStream_t s, const EPI& epi) {
  constexpr int NP = 8 / BITS, CPG = G / 32;
  const int M = (int)t->rows, N = (int)t->hidden;
  const int units = N / (32 * NP) / CPG;
  const int upb = units >= 16 ? 4 : 1;
  dim3 grid((M + 63) / 64, (units + upb - 1) / upb);
  if (t->n_outlier > 0) {
    const size_t shm = (size_t)(N / 32) * 4 + (size_t)N * 2;
    hipLaunchKernelGGL((k_decode<BITS, G, R, true, EPI>), grid, dim3(256), shm, s, (const uint8_t*)t->codes,
                       t->ld_codes, (const uint16_t*)t->scale, (const uint16_t*)t->zero, t->ld_sz,
                       (const uint16_t*)t->L, t->ld_L, (const uint16_t*)t->V, M, N, t->outlier_idx,
                       t->n_outlier, (const uint16_t*)t->side, t->ld_side, upb, epi);
  } else {
    hipLaunchKernelGGL((k_decode<BITS, G, R, false, EPI>), grid, dim3(256), 0, s, (const uint8_t*)t->codes,
                       t->ld_codes, (const uint16_t*)t->scale, (const uint16_t*)t->zero, t->ld_sz,
                       (const uint16_t*)t->L, t->ld_L, (const uint16_t*)t->V, M, N, nullptr, 0, nullptr,
                       (int64_t)0, upb, epi);
  }
  return launch_status();
}

template <class EPI>
static int decode_dispatch(const lrq_tensors* t, hipStream_t s, const EPI& epi) {
  if (t->flags & LRQ_FLAG_HADAMARD) return LRQ_ERR_UNSUPPORTED;
  switch (format_key(t->bits, t->group, t->rank)) {
    case format_key(4, 64, 0): return decode_launch<4, 64, 0>(t, s, epi);
    case format_key(4, 64, 16): return decode_launch<4, 64, 16>(t, s, epi);
    case format_key(4, 64, 32): return decode_launch<4, 64, 32>(t, s, epi);
    case format_key(4, 128, 0): return decode_launch<4, 128, 0>(t, s, epi);
    case format_key(4, 128, 16): return decode_launch<4, 128, 16>(t, s, epi);
    case format_key(8, 64, 0): return decode_launch<8, 64, 0>(t, s, epi);
    case format_key(8, 64, 16): return decode_launch<8, 64, 16>(t, s, epi);
    case format_key(8, 128, 0): return decode_launch<8, 128, 0>(t, s, epi);
    case format_key(8, 128, 16): return decode_launch<8, 128, 16>(t, s, epi);
    default: return LRQ_ERR_UNSUPPORTED;
  }
}

static int check_io(const lrq_tensors* t, const void* in, int64_t ldin, const void* out, int64_t ldout, bool need_in) {
  int st = validate_tensors(t, 0);
  if (st) return st;
  if (need_in) {
    st = validate_rows16(in, ldin, t->hidden);
    if (st) return st;
  }
  return validate_rows16(out, ldout, t->hidden);
}

}  // namespace lrq

using namespace lrq;

extern "C" int lrq_decode(const lrq_tensors* t, void* out, int64_t ldo, void* stream) {
  int st = check_io(t, nullptr, 0, out, ldo, false);
  if (st) return st;
  if (t->rows == 0) return LRQ_OK;
  return decode_dispatch(t, (hipStream_t)stream, EpiStore{(uint16_t*)out, ldo});
}

extern "C" int lrq_silu_bwd(const lrq_tensors* t, const void* dy, int64_t lddy, void* dx, int64_t lddx,
                            void* stream) {
  int st = check_io(t, dy, lddy, dx, lddx, true);
  if (st) return st;
  if (t->rows == 0) return LRQ_OK;
  return decode_dispatch(t, (hipStream_t)stream, EpiSilu{(const uint16_t*)dy, lddy, (uint16_t*)dx, lddx});
}

extern "C" int lrq_gelu_bwd(const lrq_tensors* t, const void* dy, int64_t lddy, void* dx, int64_t lddx,
                            void* stream) {
  int st = check_io(t, dy, lddy, dx, lddx, true);
  if (st) return st;
  if (t->rows == 0) return LRQ_OK;
  return decode_dispatch(t, (hipStream_t)stream, EpiGelu{(const uint16_t*)dy, lddy, (uint16_t*)dx, lddx});
}

extern "C" int lrq_mul(const lrq_tensors* t, const void* y, int64_t ldy, void* out, int64_t ldo, void* stream) {
  int st = check_io(t, y, ldy, out, ldo, true);
  if (st) return st;
  if (t->rows == 0) return LRQ_OK;
  return decode_dispatch(t, (hipStream_t)stream, EpiMul{(const uint16_t*)y, ldy, (uint16_t*)out, ldo});
}
