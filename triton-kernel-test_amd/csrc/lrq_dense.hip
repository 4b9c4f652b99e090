// Uncompressed consumers: the reference's dense Triton kernels, as streaming HIP kernels.
//
//   op 0  triton_silu_backward (silu_backward.py:54-69):    out = g * s(x) * (1 + x * (1 - s(x)))
//   op 1  triton_gelu_backward (gelu_backward.py:73-88):    tanh-approximation GELU backward
//   op 2  triton_hadamard      (extraction_fuse_hadamard.py:62-73, torch form :5-6): out = x * y
//   triton_softmax_backward    (softmax_backward.py:45-61):  out = y * (g - sum_row(g * y))
//
// All arithmetic is fp32 with one bf16 rounding of each output, as the torch library
// backward functions (aten silu_backward / gelu_backward / _softmax_backward_data) compute.
// These kernels are HBM-bound: 6 bytes per element (two bf16 reads, one bf16 write).
#include "lrq_common.h"
#include "lrq_host.h"
#include "lrq_math.h"

namespace lrq {

template <int OP>
__device__ __forceinline__ float dense_op(float x, float y) {
  if constexpr (OP == 0) return silu_bwd_f32(x, y);
  else if constexpr (OP == 1) return gelu_bwd_f32(x, y);
  else return x * y;
}

// 8 elements (16 bytes) per thread per step, grid-stride; the scalar tail covers n % 8.
template <int OP>
// out may be x (in place: each element is read and written by the same thread, reads first).
__global__ __launch_bounds__(256) void k_dense_elementwise(const uint16_t* x, const uint16_t* __restrict__ y,
                                                           uint16_t* out, int64_t n) {
  const int64_t nv = n / 8;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < nv; i += stride) {
    float a[8], b[8], o[8];
    unpack8(ld16_stream(x + 8 * i), a);
    unpack8(ld16_stream(y + 8 * i), b);
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = dense_op<OP>(a[e], b[e]);
    st16(out + 8 * i, pack8(o));
  }
  if (blockIdx.x == 0 && threadIdx.x < n - 8 * nv) {
    const int64_t k = 8 * nv + threadIdx.x;
    const float a = __uint_as_float((uint32_t)x[k] << 16), b = __uint_as_float((uint32_t)y[k] << 16);
    out[k] = (uint16_t)pack_bf16x2(dense_op<OP>(a, b), 0.f);
  }
}

// Same, for operands that are not 16-byte aligned: one element per thread.
template <int OP>
__global__ __launch_bounds__(256) void k_dense_elementwise_scalar(const uint16_t* x, const uint16_t* __restrict__ y,
                                                                  uint16_t* out, int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t k = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; k < n; k += stride) {
    const float a = __uint_as_float((uint32_t)x[k] << 16), b = __uint_as_float((uint32_t)y[k] << 16);
    out[k] = (uint16_t)pack_bf16x2(dense_op<OP>(a, b), 0.f);
  }
}

// Sum over the 256 threads of the workgroup; every thread receives it.
__device__ __forceinline__ float block_sum256(float v, float* red) {
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) v += __shfl_xor(v, m);
  const int w = threadIdx.x >> 6;
  __syncthreads();  // red may still be read by a previous call
  if ((threadIdx.x & 63) == 0) red[w] = v;
  __syncthreads();
  return (red[0] + red[1]) + (red[2] + red[3]);
}

// One workgroup per row.  VEC: the row is a whole number of 16-byte vectors and at most
// 4 per thread, so y and g stay in registers between the reduction and the output;
// otherwise one element per thread per step, with the row re-read (from L2) for the output.
template <bool VEC>
// out may be y (in place: a row's outputs are written only after every read of the row that
// precedes them in the thread, and each element by the thread that read it).
__global__ __launch_bounds__(256) void k_dense_softmax_bwd(const uint16_t* y, const uint16_t* __restrict__ g,
                                                           uint16_t* out, int64_t n) {
  __shared__ float red[4];
  const int64_t base = (int64_t)blockIdx.x * n;
  if constexpr (VEC) {
    constexpr int C = 4;
    const int nv = (int)(n / 8);
    float yv[C][8], gv[C][8];
    float acc = 0.f;
#pragma unroll
    for (int c = 0; c < C; ++c) {
      const int v = threadIdx.x + 256 * c;
      if (v < nv) {
        unpack8(ld16_stream(y + base + 8 * v), yv[c]);
        unpack8(ld16_stream(g + base + 8 * v), gv[c]);
#pragma unroll
        for (int e = 0; e < 8; ++e) acc = __builtin_fmaf(yv[c][e], gv[c][e], acc);
      }
    }
    const float s = block_sum256(acc, red);
#pragma unroll
    for (int c = 0; c < C; ++c) {
      const int v = threadIdx.x + 256 * c;
      if (v < nv) {
        float o[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = yv[c][e] * (gv[c][e] - s);
        st16(out + base + 8 * v, pack8(o));
      }
    }
  } else {
    float acc = 0.f;
    for (int64_t k = threadIdx.x; k < n; k += 256)
      acc = __builtin_fmaf(__uint_as_float((uint32_t)y[base + k] << 16), __uint_as_float((uint32_t)g[base + k] << 16), acc);
    const float s = block_sum256(acc, red);
    for (int64_t k = threadIdx.x; k < n; k += 256) {
      const float yk = __uint_as_float((uint32_t)y[base + k] << 16), gk = __uint_as_float((uint32_t)g[base + k] << 16);
      out[base + k] = (uint16_t)pack_bf16x2(yk * (gk - s), 0.f);
    }
  }
}

// extraction_outlier_channel.py:5-8: o = x * (|x| > tau), rest = x - o (tau rounded to bf16, as
// the comparison of a bf16 tensor with a scalar is evaluated).  Both exact: o is x or 0.
__global__ __launch_bounds__(256) void k_threshold_split(const uint16_t* __restrict__ x, int64_t n, float tau,
                                                         uint16_t* __restrict__ o, uint16_t* __restrict__ rest) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t k = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; k < n; k += stride) {
    const uint16_t h = x[k];
    const bool out = fabsf(__uint_as_float((uint32_t)h << 16)) > tau;
    o[k] = out ? h : (uint16_t)0;
    rest[k] = out ? (uint16_t)0 : h;
  }
}

// extraction_outlier_channel.py:11-14 (the reference indexes dim 1 of [B, M, N]):
// out[b, i, :] = x[b, idx[i], :], then x[b, idx[i], :] = 0 in place.  One workgroup per (b, i);
// indices must be distinct (a repeated index would read a row another workgroup zeroes).
__global__ __launch_bounds__(256) void k_gather_rows_zero(uint16_t* __restrict__ x, int64_t M, int64_t N,
                                                          const int32_t* __restrict__ idx, int k,
                                                          uint16_t* __restrict__ out) {
  const int64_t b = blockIdx.x / k;
  const int i = (int)(blockIdx.x - b * k);
  const int64_t m = idx[i];
  if (m < 0 || m >= M) return;
  uint16_t* src = x + (b * M + m) * N;
  uint16_t* dst = out + (b * k + i) * N;
  for (int64_t c = threadIdx.x; c < N; c += 256) {
    dst[c] = src[c];
    src[c] = 0;
  }
}

static int grid_for(int64_t work) {
  const int64_t blocks = (work + 255) / 256;
  return (int)(blocks < 1 ? 1 : (blocks > 8192 ? 8192 : blocks));
}

template <int OP>
static int dense_launch(const void* x, const void* y, void* out, int64_t n, hipStream_t s) {
  if (aligned(x, 16) && aligned(y, 16) && aligned(out, 16))
    LRQ_TRY(launch((k_dense_elementwise<OP>), dim3(grid_for(n / 8)), dim3(256), 0, s, (const uint16_t*)x,
                       (const uint16_t*)y, (uint16_t*)out, n));
  else
    LRQ_TRY(launch((k_dense_elementwise_scalar<OP>), dim3(grid_for(n)), dim3(256), 0, s, (const uint16_t*)x,
                       (const uint16_t*)y, (uint16_t*)out, n));
  return LRQ_OK;
}

}  // namespace lrq

using namespace lrq;

extern "C" int lrq_dense_elementwise(int32_t op, const void* x, const void* y, void* out, int64_t n, void* stream) {
  if (x == nullptr || y == nullptr || out == nullptr) return LRQ_ERR_NULL;
  if (n < 0) return LRQ_ERR_SHAPE;
  if (!aligned(x, 2) || !aligned(y, 2) || !aligned(out, 2)) return LRQ_ERR_ALIGN;
  if (n == 0) return LRQ_OK;
  hipStream_t s = (hipStream_t)stream;
  switch (op) {
    case 0: return dense_launch<0>(x, y, out, n, s);
    case 1: return dense_launch<1>(x, y, out, n, s);
    case 2: return dense_launch<2>(x, y, out, n, s);
    default: return LRQ_ERR_UNSUPPORTED;
  }
}

extern "C" int lrq_dense_softmax_bwd(const void* y, const void* g, void* out, int64_t rows, int64_t n_cols,
                                     void* stream) {
  if (y == nullptr || g == nullptr || out == nullptr) return LRQ_ERR_NULL;
  if (rows < 0 || n_cols <= 0 || rows > INT32_MAX) return LRQ_ERR_SHAPE;
  if (!aligned(y, 2) || !aligned(g, 2) || !aligned(out, 2)) return LRQ_ERR_ALIGN;
  if (rows == 0) return LRQ_OK;
  hipStream_t s = (hipStream_t)stream;
  const bool vec = n_cols % 8 == 0 && n_cols <= 256 * 8 * 4 && aligned(y, 16) && aligned(g, 16) && aligned(out, 16);
  if (vec)
    LRQ_TRY(launch((k_dense_softmax_bwd<true>), dim3((unsigned)rows), dim3(256), 0, s, (const uint16_t*)y,
                       (const uint16_t*)g, (uint16_t*)out, n_cols));
  else
    LRQ_TRY(launch((k_dense_softmax_bwd<false>), dim3((unsigned)rows), dim3(256), 0, s, (const uint16_t*)y,
                       (const uint16_t*)g, (uint16_t*)out, n_cols));
  return LRQ_OK;
}

extern "C" int lrq_threshold_split(const void* x, int64_t n, float threshold, void* outlier, void* rest,
                                   void* stream) {
  if (x == nullptr || outlier == nullptr || rest == nullptr) return LRQ_ERR_NULL;
  if (n < 0) return LRQ_ERR_SHAPE;
  if (!aligned(x, 2) || !aligned(outlier, 2) || !aligned(rest, 2)) return LRQ_ERR_ALIGN;
  if (n == 0) return LRQ_OK;
  const float tau = bf16_value_host(bf16_bits_host(threshold));
  LRQ_TRY(launch(k_threshold_split, dim3(grid_for(n)), dim3(256), 0, (hipStream_t)stream, (const uint16_t*)x, n, tau,
                     (uint16_t*)outlier, (uint16_t*)rest));
  return LRQ_OK;
}

extern "C" int lrq_gather_rows_zero(void* x, int64_t B, int64_t M, int64_t N, const int32_t* idx, int32_t k,
                                    void* out, void* stream) {
  if (x == nullptr || (k > 0 && (idx == nullptr || out == nullptr))) return LRQ_ERR_NULL;
  if (B < 0 || M < 0 || N < 0 || k < 0 || B * (int64_t)k > INT32_MAX) return LRQ_ERR_SHAPE;
  if (!aligned(x, 2) || (out != nullptr && !aligned(out, 2)) || (idx != nullptr && !aligned(idx, 4))) return LRQ_ERR_ALIGN;
  if (B == 0 || k == 0 || N == 0) return LRQ_OK;
  LRQ_TRY(launch(k_gather_rows_zero, dim3((unsigned)(B * k)), dim3(256), 0, (hipStream_t)stream, (uint16_t*)x, M, N,
                     idx, (int)k, (uint16_t*)out));
  return LRQ_OK;
}
