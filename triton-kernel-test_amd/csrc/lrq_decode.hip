// Group-mode decode and the fused elementwise consumers (SiLU backward, GELU backward,
// elementwise product).  One streaming pass: codes, qparams and L are read once, the
// low-rank term L V^T is rebuilt on MFMA in the lanes that own the columns, and the
// epilogue either stores x_hat (bf16) or applies the consumer with the
// upstream gradient, so the full-precision activation never goes back to HBM.
//
// Work split: a workgroup is NW waves on NW consecutive units (G columns of every packing
// plane, see lrq_common.h) of the same rows; each wave keeps its unit's V operands in
// registers and walks its row blocks, prefetching the next block's codes, qparams and L
// while it computes the current.
#include "lrq_common.h"
#include "lrq_host.h"

namespace lrq {

// ------------------------------------------------------------------ epilogues
// An epilogue binds its row pointers once per row block (`row(r)`), then receives 8
// consecutive reconstructed values (fp32, before the bf16 rounding that defines x_hat)
// for columns col .. col + 7 of that row.  Stores are unconditional: lanes of rows past the
// end are clamped to the last row and store the same bytes as its own lanes, which keeps
// the instruction stream branch-free (on gfx9 a conditional store makes the compiler drain
// every outstanding memory operation at the next load use, prefetches included).
struct EpiStore {
  uint16_t* out;
  int64_t ld;
  struct Row {
    uint16_t* o;
  };
  __device__ __forceinline__ Row row(int64_t r) const { return Row{out + r * ld}; }
  __device__ __forceinline__ void operator()(const Row& r, int col, const float* xh) const {
    st16(r.o + col, pack8(xh));
  }
};

struct RowIO {
  const uint16_t* in;
  uint16_t* o;
};

// silu_backward.py:6-8: dy * (s * (1 + x * (1 - s))), s = sigmoid(x), x = bf16(x_hat); fp32.
struct EpiSilu {
  const uint16_t* dy;
  int64_t lddy;
  uint16_t* dx;
  int64_t lddx;
  using Row = RowIO;
  __device__ __forceinline__ Row row(int64_t r) const { return Row{dy + r * lddy, dx + r * lddx}; }
  __device__ __forceinline__ void operator()(const Row& r, int col, const float* xh) const {
    float d[8], o[8];
    unpack8(ld16_stream(r.in + col), d);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float x = bf16_roundtrip(xh[e]);
      const float s = __builtin_amdgcn_rcpf(1.f + __expf(-x));
      o[e] = d[e] * (s * (1.f + x * (1.f - s)));
    }
    st16(r.o + col, pack8(o));
  }
};

// gelu_backward.py:14-21 (tanh approximation), fp32 on x = bf16(x_hat).
struct EpiGelu {
  const uint16_t* dy;
  int64_t lddy;
  uint16_t* dx;
  int64_t lddx;
  using Row = RowIO;
  __device__ __forceinline__ Row row(int64_t r) const { return Row{dy + r * lddy, dx + r * lddx}; }
  __device__ __forceinline__ void operator()(const Row& r, int col, const float* xh) const {
    constexpr float kGamma = 0.7978845608028654f, kKappa = 0.044715f;
    float d[8], o[8];
    unpack8(ld16_stream(r.in + col), d);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float x = bf16_roundtrip(xh[e]);
      const float x2 = x * x;
      const float u = kGamma * (x + kKappa * x2 * x);
      // tanh(u) = 1 - 2 / (exp(2u) + 1); saturates correctly at +-1.
      const float th = 1.f - 2.f * __builtin_amdgcn_rcpf(__expf(2.f * u) + 1.f);
      o[e] = 0.5f * ((1.f + th) + x * ((1.f - th * th) * kGamma * (1.f + 3.f * kKappa * x2))) * d[e];
    }
    st16(r.o + col, pack8(o));
  }
};

// extraction_fuse_hadamard.py:5-6: x * y.
struct EpiMul {
  const uint16_t* y;
  int64_t ldy;
  uint16_t* out;
  int64_t ldo;
  using Row = RowIO;
  __device__ __forceinline__ Row row(int64_t r) const { return Row{y + r * ldy, out + r * ldo}; }
  __device__ __forceinline__ void operator()(const Row& r, int col, const float* xh) const {
    float a[8], o[8];
    unpack8(ld16_stream(r.in + col), a);
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = bf16_roundtrip(xh[e]) * a[e];
    st16(r.o + col, pack8(o));
  }
};

// ------------------------------------------------------------------ kernel
// Per-row-block inputs of one lane: its G/4 code bytes, the unit's NP (scale, zero) pairs
// and the L operand of its row.
template <int BITS, int G, int R>
struct DecIn {
  u32x4 cb[G / 64];
  uint32_t qp[8 / BITS];
  u32x2 lop[R > 0 ? R / 16 : 1];
};

// Grid: (ceil(row blocks / RBW), ceil(units / NW)); NW waves; wave w owns unit
// blockIdx.y * NW + w and walks row blocks blockIdx.x * RBW + b, b < RBW.  The waves of a
// workgroup work on consecutive units of the same rows, so at any time a workgroup writes
// NW * G * 2 contiguous bytes per row and plane (DRAM-page friendly), while each wave
// reuses its unit's V operands for all its row blocks.
template <int BITS, int G, int R, bool OUTL, int NW, int RBW, class EPI>
__global__ __launch_bounds__(NW * 64) void k_decode(
    const uint8_t* __restrict__ codes, int64_t ldc, const uint16_t* __restrict__ qparams, int64_t ldq,
    const uint16_t* __restrict__ Lin, int64_t ldl, const uint16_t* __restrict__ V, int M, int N,
    const int32_t* __restrict__ oidx, int nout, const uint16_t* __restrict__ side, int64_t ldside,
    EPI epi) {
  constexpr int NP = 8 / BITS, RT = R > 0 ? R / 16 : 1, E = G / 4;
  constexpr uint32_t kMask = (1u << BITS) - 1u;
  extern __shared__ uint32_t smem[];
  uint32_t* colmask = smem;                                    // N/32 words
  int16_t* slot = reinterpret_cast<int16_t*>(smem + N / 32);  // N entries
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
  const int u = blockIdx.y * NW + w;
  if (u >= N / (G * NP)) return;  // tail workgroup of a row: idle wave (no barrier follows)
  const int nrb = (M + 15) / 16;

  u32x2 vop[NP][G / 16][RT];
  if constexpr (R > 0) {
#pragma unroll
    for (int p = 0; p < NP; ++p) load_vops<G, R>(V, unit_base(p, u, N, NP, G), j, g, vop[p]);
  }

  auto load = [&](DecIn<BITS, G, R>& in, int rb, bool valid) {
    const int64_t row = valid ? min(rb * 16 + j, M - 1) : 0;
    const uint8_t* cp = codes + row * ldc + u * G + E * g;
#pragma unroll
    for (int i = 0; i < G / 64; ++i) in.cb[i] = ld16_stream(cp + 16 * i);
    const uint16_t* qpp = qparams + row * ldq + u * NP * 2;
    if constexpr (NP == 2) {
      const u32x2 v = ld8(qpp);
      in.qp[0] = v[0];
      in.qp[1] = v[1];
    } else {
      in.qp[0] = ld4(qpp);
    }
    if constexpr (R > 0) {
#pragma unroll
      for (int t = 0; t < RT; ++t) in.lop[t] = ld8(Lin + row * ldl + 16 * t + 4 * g);
    }
  };

  auto compute = [&](const DecIn<BITS, G, R>& in, int rb) {
    const int64_t rr = min(rb * 16 + j, M - 1);
    const typename EPI::Row erow = epi.row(rr);
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      const float sf = f16_val(in.qp[p] & 0xffffu);
      const float zf = f16_val(in.qp[p] >> 16);
      float xh[E];
#pragma unroll
      for (int d = 0; d < E / 4; ++d) {
        // the codes of plane p for elements 4d .. 4d+3, one per byte
        const uint32_t wd = in.cb[d >> 2][d & 3];
        const uint32_t wq = NP == 1 ? wd : ((wd >> (BITS * p)) & (0x01010101u * kMask));
        // code * scale is exact, so the fma rounds once, like the oracle's mul + add
        xh[4 * d + 0] = __builtin_fmaf(ubyte_f32<0>(wq), sf, zf);
        xh[4 * d + 1] = __builtin_fmaf(ubyte_f32<1>(wq), sf, zf);
        xh[4 * d + 2] = __builtin_fmaf(ubyte_f32<2>(wq), sf, zf);
        xh[4 * d + 3] = __builtin_fmaf(ubyte_f32<3>(wq), sf, zf);
      }
      if constexpr (R > 0) residual_unit<G, R>(vop[p], in.lop, xh, xh);  // d + L V^T, one rounding
      const int c0 = unit_base(p, u, N, NP, G) + E * g;
      if constexpr (OUTL) {
        const uint32_t mbits = colmask[c0 >> 5] >> (c0 & 31);
        if (mbits != 0u) {
#pragma unroll
          for (int e = 0; e < E; ++e)
            if ((mbits >> e) & 1u) xh[e] = f16_val(side[rr * ldside + slot[c0 + e]]);
        }
      }
#pragma unroll
      for (int k = 0; k < E / 8; ++k) epi(erow, c0 + 8 * k, xh + 8 * k);
    }
  };

  const int rb0 = blockIdx.x * RBW;
  if (rb0 >= nrb) return;
  // All of the wave's row-block inputs are requested up front (codes, qparams and L are a
  // quarter of the traffic); blocks are then reconstructed and stored in order.  With RBW a
  // compile-time constant and no branch in the body every wait count is exact and no load
  // is issued after a store.  Blocks past the end (tail workgroup only) repeat the last row
  // block, rewriting the same bytes.
  DecIn<BITS, G, R> in[RBW];
#pragma unroll
  for (int b = 0; b < RBW; ++b) load(in[b], min(rb0 + b, nrb - 1), true);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int b = 0; b < RBW; ++b) compute(in[b], min(rb0 + b, nrb - 1));
}

// ------------------------------------------------------------------ host side
template <int BITS, int G, int R, int RBW, class EPI>
static int decode_launch_rbw(const lrq_tensors* t, hipStream_t s, const EPI& epi) {
  constexpr int NP = 8 / BITS, NW = 8;
  const int M = (int)t->rows, N = (int)t->hidden;
  const int units = N / (G * NP);
  const int nrb = (M + 15) / 16;
  dim3 grid((nrb + RBW - 1) / RBW, (units + NW - 1) / NW);
  if (t->n_outlier > 0) {
    const size_t shm = (size_t)(N / 32) * 4 + (size_t)N * 2;
    hipLaunchKernelGGL((k_decode<BITS, G, R, true, NW, RBW, EPI>), grid, dim3(NW * 64), shm, s,
                       (const uint8_t*)t->codes, t->ld_codes, (const uint16_t*)t->qparams, t->ld_qp,
                       (const uint16_t*)t->L, t->ld_L, (const uint16_t*)t->V, M, N, t->outlier_idx, t->n_outlier,
                       (const uint16_t*)t->side, t->ld_side, epi);
  } else {
    hipLaunchKernelGGL((k_decode<BITS, G, R, false, NW, RBW, EPI>), grid, dim3(NW * 64), 0, s,
                       (const uint8_t*)t->codes, t->ld_codes, (const uint16_t*)t->qparams, t->ld_qp,
                       (const uint16_t*)t->L, t->ld_L, (const uint16_t*)t->V, M, N, nullptr, 0, nullptr,
                       (int64_t)0, epi);
  }
  return launch_status();
}

// 8 row blocks per wave when that still leaves >= 512 workgroups (2 per CU), else 2.
template <int BITS, int G, int R, class EPI>
static int decode_launch(const lrq_tensors* t, hipStream_t s, const EPI& epi) {
  constexpr int NP = 8 / BITS, NW = 8;
  const int64_t units = t->hidden / (G * NP), nrb = (t->rows + 15) / 16;
  const int64_t wgs8 = ((nrb + 7) / 8) * ((units + NW - 1) / NW);
  if (wgs8 >= 512) return decode_launch_rbw<BITS, G, R, 8>(t, s, epi);
  return decode_launch_rbw<BITS, G, R, 2>(t, s, epi);
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

static int check_io(const lrq_tensors* t, const void* in, int64_t ldin, const void* out, int64_t ldout,
                    bool need_in) {
  int st = validate_tensors(t);
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
