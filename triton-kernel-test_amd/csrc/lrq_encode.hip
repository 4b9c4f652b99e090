// Group-mode encode: projection L = bf16(X V), residual R = X - L V^T, per-group
// asymmetric quantisation and row-planar packing.
//
// Two implementations, chosen per call by lrq_encode():
//   * k_encode_fused — one pass over X.  A workgroup owns 16 full rows; its NW waves
//     split the hidden dimension and keep their share of X in registers (the row is
//     needed twice: once for the projection, once for the residual, and only a whole
//     row gives L).  Partial L tiles are reduced across waves through LDS.  Instantiated
//     for the hidden sizes listed in encode_fused_dispatch().
//   * k_project + k_quant — two passes for any other hidden size (and rank 0 without
//     the projection): X is read twice.
#include "lrq_common.h"
#include "lrq_quant.h"
#include "lrq_host.h"

namespace lrq {

// -------------------------------------------------------------------------------------
// Single-pass encode.  Grid: ceil(rows / 16) workgroups of NW waves.  Wave w owns chunks
// [w*CPW, (w+1)*CPW) of every packing plane; the host guarantees hidden == NW*CPW*32*NP.
template <int BITS, int G, int R, int NW, int CPW>
__global__ __launch_bounds__(NW * 64) void k_encode_fused(
    const uint16_t* __restrict__ X, int64_t ldx, int M, int N, const uint16_t* __restrict__ V,
    const uint16_t* __restrict__ Vt, uint16_t* __restrict__ Lout, int64_t ldl,
    uint8_t* __restrict__ codes, int64_t ldc, uint16_t* __restrict__ scale,
    uint16_t* __restrict__ zero, int64_t ldsz) {
  constexpr int NP = 8 / BITS, CPG = G / 32, RT = R / 16;
  static_assert(CPW % CPG == 0, "a wave must own whole groups");
  constexpr int PC = NW * CPW;  // chunks per plane
  __shared__ f32x4 red[NW * RT * 64];

  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int j = lane & 15, g = lane >> 4;
  const int row = blockIdx.x * 16 + j;
  const bool rv = row < M;
  const uint16_t* xrow = X + (int64_t)(rv ? row : 0) * ldx;

  u32x4 xr[NP][CPW];
#pragma unroll
  for (int p = 0; p < NP; ++p)
#pragma unroll
    for (int k = 0; k < CPW; ++k) {
      const int col = (p * PC + w * CPW + k) * 32 + 8 * g;
      xr[p][k] = rv ? ld16_stream(xrow + col) : u32x4{0u, 0u, 0u, 0u};
    }

  // Projection, transposed: D(rank, row) += Vt(rank, cols) * X^T(cols, row).  Lane (j, g)
  // ends up with L[row j][16t + 4g + v], v = 0..3 — the B-operand layout of the residual.
  f32x4 acc[RT];
#pragma unroll
  for (int t = 0; t < RT; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int p = 0; p < NP; ++p)
#pragma unroll
    for (int k = 0; k < CPW; ++k) {
      const int col = (p * PC + w * CPW + k) * 32 + 8 * g;
#pragma unroll
      for (int t = 0; t < RT; ++t) {
        const u32x4 a = ld16(Vt + (int64_t)(16 * t + j) * N + col);
        acc[t] = mfma_16x16x32(a, xr[p][k], acc[t]);
      }
    }
#pragma unroll
  for (int t = 0; t < RT; ++t) red[(w * RT + t) * 64 + lane] = acc[t];
  __syncthreads();
  u32x2 lop[RT];
#pragma unroll
  for (int t = 0; t < RT; ++t) {
    f32x4 s = red[t * 64 + lane];
#pragma unroll
    for (int w2 = 1; w2 < NW; ++w2) {
      const f32x4 o = red[(w2 * RT + t) * 64 + lane];
      s[0] += o[0];
      s[1] += o[1];
      s[2] += o[2];
      s[3] += o[3];
    }
    lop[t] = u32x2{pack_bf16x2(s[0], s[1]), pack_bf16x2(s[2], s[3])};
    if (w == 0 && rv) st8(Lout + (int64_t)row * ldl + 16 * t + 4 * g, lop[t]);
  }

  uint8_t* crow = codes + (int64_t)row * ldc;
  uint16_t* srow = scale + (int64_t)row * ldsz;
  uint16_t* zrow = zero + (int64_t)row * ldsz;
#pragma unroll
  for (int u = 0; u < CPW / CPG; ++u) {
    u32x4 xu[NP][CPG];
#pragma unroll
    for (int p = 0; p < NP; ++p)
#pragma unroll
      for (int k = 0; k < CPG; ++k) xu[p][k] = xr[p][u * CPG + k];
    quant_unit<BITS, G, R>(xu, w * CPW + u * CPG, PC, V, lop, nullptr, j, g, rv, crow, srow, zrow);
  }
}

// -------------------------------------------------------------------------------------
// Projection only (first pass of the two-pass encode).  Grid: ceil(rows / 16) workgroups
// of 4 waves; wave w sums chunks w, w + 4, ... of the row.
template <int R>
__global__ __launch_bounds__(256) void k_project(const uint16_t* __restrict__ X, int64_t ldx, int M,
                                                 int N, const uint16_t* __restrict__ Vt,
                                                 uint16_t* __restrict__ Lout, int64_t ldl) {
  constexpr int RT = R / 16, U = 4, NWV = 4;
  __shared__ f32x4 red[NWV * RT * 64];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int j = lane & 15, g = lane >> 4;
  const int row = blockIdx.x * 16 + j;
  const bool rv = row < M;
  const uint16_t* xrow = X + (int64_t)(rv ? row : 0) * ldx;
  const int NC = N / 32;
  f32x4 acc[RT];
#pragma unroll
  for (int t = 0; t < RT; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int c = w; c < NC; c += NWV * U) {
    u32x4 xv[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int cc = c + NWV * u;
      xv[u] = (cc < NC && rv) ? ld16_stream(xrow + cc * 32 + 8 * g) : u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int cc = c + NWV * u;
      if (cc < NC) {
#pragma unroll
        for (int t = 0; t < RT; ++t) {
          const u32x4 a = ld16(Vt + (int64_t)(16 * t + j) * N + cc * 32 + 8 * g);
          acc[t] = mfma_16x16x32(a, xv[u], acc[t]);
        }
      }
    }
  }
#pragma unroll
  for (int t = 0; t < RT; ++t) red[(w * RT + t) * 64 + lane] = acc[t];
  __syncthreads();
  if (w == 0) {
#pragma unroll
    for (int t = 0; t < RT; ++t) {
      f32x4 s = red[t * 64 + lane];
#pragma unroll
      for (int w2 = 1; w2 < NWV; ++w2) {
        const f32x4 o = red[(w2 * RT + t) * 64 + lane];
        s[0] += o[0];
        s[1] += o[1];
        s[2] += o[2];
        s[3] += o[3];
      }
      if (rv)
        st8(Lout + (int64_t)row * ldl + 16 * t + 4 * g,
            u32x2{pack_bf16x2(s[0], s[1]), pack_bf16x2(s[2], s[3])});
    }
  }
}

// -------------------------------------------------------------------------------------
// Streaming residual + quantisation (second pass; also the whole encode at rank 0).
// Grid: (ceil(rows / 64), ceil(units / upb)); a workgroup is 4 waves x 16 rows and walks
// `upb` units.  With OUTL, outlier columns are zeroed before the group statistics.
template <int BITS, int G, int R, bool OUTL>
__global__ __launch_bounds__(256) void k_quant(
    const uint16_t* __restrict__ X, int64_t ldx, int M, int N, const uint16_t* __restrict__ V,
    const uint16_t* __restrict__ Lin, int64_t ldl, uint8_t* __restrict__ codes, int64_t ldc,
    uint16_t* __restrict__ scale, uint16_t* __restrict__ zero, int64_t ldsz,
    const int32_t* __restrict__ oidx, int nout, int upb) {
  constexpr int NP = 8 / BITS, CPG = G / 32, RT = R > 0 ? R / 16 : 1;
  extern __shared__ uint32_t colmask[];
  const int PC = N / (32 * NP);
  const int units = PC / CPG;
  if constexpr (OUTL) {
    for (int i = threadIdx.x; i < N / 32; i += blockDim.x) colmask[i] = 0u;
    __syncthreads();
    for (int k = threadIdx.x; k < nout; k += blockDim.x) {
      const int c = oidx[k];
      if (c >= 0 && c < N) atomicOr(&colmask[c >> 5], 1u << (c & 31));
    }
    __syncthreads();
  }
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int j = lane & 15, g = lane >> 4;
  const int row = blockIdx.x * 64 + w * 16 + j;
  const bool rv = row < M;
  const int64_t rr = rv ? row : 0;
  const uint16_t* xrow = X + rr * ldx;
  u32x2 lop[RT];
  if constexpr (R > 0) {
#pragma unroll
    for (int t = 0; t < RT; ++t)
      lop[t] = rv ? ld8(Lin + rr * ldl + 16 * t + 4 * g) : u32x2{0u, 0u};
  }
  uint8_t* crow = codes + rr * ldc;
  uint16_t* srow = scale + rr * ldsz;
  uint16_t* zrow = zero + rr * ldsz;
  for (int ui = 0; ui < upb; ++ui) {
    const int u = blockIdx.y * upb + ui;
    if (u >= units) break;
    const int cu = u * CPG;
    u32x4 xu[NP][CPG];
#pragma unroll
    for (int p = 0; p < NP; ++p)
#pragma unroll
      for (int k = 0; k < CPG; ++k)
        xu[p][k] = rv ? ld16_stream(xrow + (p * PC + cu + k) * 32 + 8 * g) : u32x4{0u, 0u, 0u, 0u};
    quant_unit<BITS, G, R>(xu, cu, PC, V, lop, OUTL ? colmask : nullptr, j, g, rv, crow, srow, zrow);
  }
}

// Gather the outlier channels into fp16 side columns: side[r, k] = fp16(x[r, idx[k]]).
__global__ __launch_bounds__(256) void k_gather_side(const uint16_t* __restrict__ X, int64_t ldx, int M,
                                                     int N, const int32_t* __restrict__ oidx, int nout,
                                                     uint16_t* __restrict__ side, int64_t ldside) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (int64_t)M * nout) return;
  const int64_t r = i / nout;
  const int k = (int)(i - r * nout);
  const int c = oidx[k];
  const float v = (c >= 0 && c < N) ? __uint_as_float((uint32_t)X[r * ldx + c] << 16) : 0.f;
  side[r * ldside + k] = f16_bits(v);
}

// -------------------------------------------------------------------------------------
// host side

template <int BITS, int G, int R, int NW, int CPW>
static int launch_fused(const lrq_tensors* t, const void* x, int64_t ldx, hipStream_t s) {
  dim3 grid((unsigned)((t->rows + 15) / 16));
  hipLaunchKernelGGL((k_encode_fused<BITS, G, R, NW, CPW>), grid, dim3(NW * 64), 0, s,
                     (const uint16_t*)x, ldx, (int)t->rows, (int)t->hidden, (const uint16_t*)t->V,
                     (const uint16_t*)t->Vt, (uint16_t*)t->L, t->ld_L, (uint8_t*)t->codes, t->ld_codes,
                     (uint16_t*)t->scale, (uint16_t*)t->zero, t->ld_sz);
  return launch_status();
}

template <int BITS, int G, int R, int NW, int CPW>
static int try_fused(const lrq_tensors* t, const void* x, int64_t ldx, hipStream_t s, int* status) {
  if constexpr (CPW % (G / 32) == 0) {
    *status = launch_fused<BITS, G, R, NW, CPW>(t, x, ldx, s);
    return 1;
  } else {
    return 0;
  }
}

// Returns 1 and launches when a single-pass kernel exists for this shape, else 0.
// Chunks per plane (pc) = hidden / (32 * NP) is split over NW waves of CPW chunks.
template <int BITS, int G, int R>
static int encode_fused_dispatch(const lrq_tensors* t, const void* x, int64_t ldx, hipStream_t s,
                                 int* status) {
  constexpr int NP = 8 / BITS;
  const int64_t pc = t->hidden / (32 * NP);
  switch (pc) {
    case 16: return try_fused<BITS, G, R, 4, 4>(t, x, ldx, s, status);
    case 32: return try_fused<BITS, G, R, 4, 8>(t, x, ldx, s, status);
    case 64: return try_fused<BITS, G, R, 8, 8>(t, x, ldx, s, status);
    case 80: return try_fused<BITS, G, R, 8, 10>(t, x, ldx, s, status);
    default: return 0;
  }
}

template <int BITS, int G, int R>
static int encode_twopass(const lrq_tensors* t, const void* x, int64_t ldx, hipStream_t s) {
  const int M = (int)t->rows, N = (int)t->hidden;
  constexpr int NP = 8 / BITS, CPG = G / 32;
  if constexpr (R > 0) {
    hipLaunchKernelGGL((k_project<R>), dim3((M + 15) / 16), dim3(256), 0, s, (const uint16_t*)x, ldx, M,
                       N, (const uint16_t*)t->Vt, (uint16_t*)t->L, t->ld_L);
    int st = launch_status();
    if (st) return st;
  }
  const int units = N / (32 * NP) / CPG;
  const int upb = 4;
  dim3 grid((M + 63) / 64, (units + upb - 1) / upb);
  const bool outl = t->n_outlier > 0;
  if (outl) {
    hipLaunchKernelGGL((k_quant<BITS, G, R, true>), grid, dim3(256), (size_t)(N / 32) * 4, s,
                       (const uint16_t*)x, ldx, M, N, (const uint16_t*)t->V, (const uint16_t*)t->L, t->ld_L,
                       (uint8_t*)t->codes, t->ld_codes, (uint16_t*)t->scale, (uint16_t*)t->zero, t->ld_sz,
                       t->outlier_idx, t->n_outlier, upb);
    int st = launch_status();
    if (st) return st;
    const int64_t n = (int64_t)M * t->n_outlier;
    hipLaunchKernelGGL(k_gather_side, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, (const uint16_t*)x,
                       ldx, M, N, t->outlier_idx, t->n_outlier, (uint16_t*)t->side, t->ld_side);
  } else {
    hipLaunchKernelGGL((k_quant<BITS, G, R, false>), grid, dim3(256), 0, s, (const uint16_t*)x, ldx, M, N,
                       (const uint16_t*)t->V, (const uint16_t*)t->L, t->ld_L, (uint8_t*)t->codes,
                       t->ld_codes, (uint16_t*)t->scale, (uint16_t*)t->zero, t->ld_sz, nullptr, 0, upb);
  }
  return launch_status();
}

template <int BITS, int G, int R>
static int encode_impl(const lrq_tensors* t, const void* x, int64_t ldx, hipStream_t s, int force_twopass) {
  if constexpr (R > 0) {
    int st = 0;
    if (!force_twopass && t->n_outlier == 0 && encode_fused_dispatch<BITS, G, R>(t, x, ldx, s, &st)) return st;
  }
  return encode_twopass<BITS, G, R>(t, x, ldx, s);
}

static int encode_entry(const lrq_tensors* t, const void* x, int64_t ldx, void* stream, int force_twopass) {
  int st = validate_tensors(t, /*encode=*/1);
  if (st) return st;
  if (x == nullptr) return LRQ_ERR_NULL;
  if (ldx < t->hidden || (ldx % 8) != 0 || !aligned(x, 16)) return ldx < t->hidden ? LRQ_ERR_SHAPE : LRQ_ERR_ALIGN;
  if (t->rows == 0) return LRQ_OK;
  hipStream_t s = (hipStream_t)stream;
  const int key = format_key(t->bits, t->group, t->rank);
  switch (key) {
    case format_key(4, 64, 0): return encode_impl<4, 64, 0>(t, x, ldx, s, force_twopass);
    case format_key(4, 64, 16): return encode_impl<4, 64, 16>(t, x, ldx, s, force_twopass);
    case format_key(4, 64, 32): return encode_impl<4, 64, 32>(t, x, ldx, s, force_twopass);
    case format_key(4, 128, 0): return encode_impl<4, 128, 0>(t, x, ldx, s, force_twopass);
    case format_key(4, 128, 16): return encode_impl<4, 128, 16>(t, x, ldx, s, force_twopass);
    case format_key(8, 64, 0): return encode_impl<8, 64, 0>(t, x, ldx, s, force_twopass);
    case format_key(8, 64, 16): return encode_impl<8, 64, 16>(t, x, ldx, s, force_twopass);
    case format_key(8, 128, 0): return encode_impl<8, 128, 0>(t, x, ldx, s, force_twopass);
    case format_key(8, 128, 16): return encode_impl<8, 128, 16>(t, x, ldx, s, force_twopass);
    default: return LRQ_ERR_UNSUPPORTED;
  }
}

}  // namespace lrq

extern "C" int lrq_encode(const lrq_tensors* t, const void* x, int64_t ldx, void* stream) {
  return lrq::encode_entry(t, x, ldx, stream, 0);
}

// Test hook: the two-pass path for shapes that also have a single-pass kernel.
extern "C" int lrq_encode_twopass(const lrq_tensors* t, const void* x, int64_t ldx, void* stream) {
  return lrq::encode_entry(t, x, ldx, stream, 1);
}
