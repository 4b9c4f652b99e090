// Small helpers on the path: bf16 transpose (basis layouts), column abs-max and top-k
// channel selection for the outlier-channel split, status strings.
#include "lrq_common.h"
#include "lrq_host.h"

namespace lrq {

// dst[c, r] = src[r, c]; 32x32 tiles through LDS (bank-conflict-free with the +1 pad).
__global__ __launch_bounds__(256) void k_transpose_bf16(const uint16_t* __restrict__ src, int64_t rows,
                                                        int64_t cols, uint16_t* __restrict__ dst) {
  __shared__ uint16_t tile[32][33];
  const int64_t r0 = (int64_t)blockIdx.y * 32, c0 = (int64_t)blockIdx.x * 32;
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;  // 8 rows per pass
  for (int i = ty; i < 32; i += 8) {
    const int64_t r = r0 + i, c = c0 + tx;
    if (r < rows && c < cols) tile[i][tx] = src[r * cols + c];
  }
  __syncthreads();
  for (int i = ty; i < 32; i += 8) {
    const int64_t c = c0 + i, r = r0 + tx;
    if (r < rows && c < cols) dst[c * rows + r] = tile[tx][i];
  }
}

// colmax[c] = max |x[r, c]| via an unsigned max on the fp32 bit pattern (valid for
// non-negative floats).  colmax must be zeroed first (done by the host entry).
// Grid: (ceil(cols / 512), ceil(rows / 64)); each thread owns 2 adjacent columns and
// walks 64 rows.
__global__ __launch_bounds__(256) void k_colmax(const uint16_t* __restrict__ x, int64_t ldx, int64_t rows,
                                                int64_t cols, unsigned int* __restrict__ colmax) {
  const int64_t c = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 2;
  if (c >= cols) return;
  const int64_t r0 = (int64_t)blockIdx.y * 64;
  const int64_t r1 = r0 + 64 < rows ? r0 + 64 : rows;
  float m0 = 0.f, m1 = 0.f;
  for (int64_t r = r0; r < r1; ++r) {
    const uint32_t v = *reinterpret_cast<const uint32_t*>(x + r * ldx + c);
    m0 = fmaxf(m0, fabsf(bf_lo(v)));
    m1 = fmaxf(m1, fabsf(bf_hi(v)));
  }
  atomicMax(colmax + c, __float_as_uint(m0));
  atomicMax(colmax + c + 1, __float_as_uint(m1));
}

__global__ void k_zero_u32(unsigned int* p, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0u;
}

// Top-k by repeated block argmax in one 1024-thread workgroup (k is small: tens of
// channels).  Ties go to the lower column index.  Output sorted ascending.
// LDS: hidden floats (value copy) + 1024 (value, index) reduction slots.
__global__ __launch_bounds__(1024) void k_topk(const float* __restrict__ colmax, int hidden, int k,
                                               int32_t* __restrict__ idx) {
  extern __shared__ float sval[];
  float* rv = sval + hidden;
  int* ri = reinterpret_cast<int*>(rv + 1024);
  int* picked = ri + 1024;
  for (int i = threadIdx.x; i < hidden; i += blockDim.x) sval[i] = colmax[i];
  __syncthreads();
  for (int it = 0; it < k; ++it) {
    float bv = -1.f;
    int bi = 0x7fffffff;
    for (int i = threadIdx.x; i < hidden; i += blockDim.x) {
      const float v = sval[i];
      if (v > bv || (v == bv && i < bi)) {
        bv = v;
        bi = i;
      }
    }
    rv[threadIdx.x] = bv;
    ri[threadIdx.x] = bi;
    __syncthreads();
    for (int s = 512; s > 0; s >>= 1) {
      if ((int)threadIdx.x < s) {
        const float ov = rv[threadIdx.x + s];
        const int oi = ri[threadIdx.x + s];
        if (ov > rv[threadIdx.x] || (ov == rv[threadIdx.x] && oi < ri[threadIdx.x])) {
          rv[threadIdx.x] = ov;
          ri[threadIdx.x] = oi;
        }
      }
      __syncthreads();
    }
    if (threadIdx.x == 0) {
      picked[it] = ri[0];
      sval[ri[0]] = -2.f;  // below every |x|
    }
    __syncthreads();
  }
  // rank-sort the k picked indices ascending
  for (int a = threadIdx.x; a < k; a += blockDim.x) {
    const int v = picked[a];
    int pos = 0;
    for (int b = 0; b < k; ++b) pos += picked[b] < v;
    idx[pos] = v;
  }
}

}  // namespace lrq

using namespace lrq;

extern "C" int lrq_transpose_bf16(const void* src, int64_t rows, int64_t cols, void* dst, void* stream) {
  if (src == nullptr || dst == nullptr) return LRQ_ERR_NULL;
  if (rows < 0 || cols < 0) return LRQ_ERR_SHAPE;
  if (!aligned(src, 2) || !aligned(dst, 2)) return LRQ_ERR_ALIGN;
  if (rows == 0 || cols == 0) return LRQ_OK;
  dim3 grid((unsigned)((cols + 31) / 32), (unsigned)((rows + 31) / 32));
  hipLaunchKernelGGL(k_transpose_bf16, grid, dim3(256), 0, (hipStream_t)stream, (const uint16_t*)src, rows,
                     cols, (uint16_t*)dst);
  return launch_status();
}

extern "C" int lrq_colmax(const void* x, int64_t ldx, int64_t rows, int64_t hidden, float* colmax,
                          void* stream) {
  if (x == nullptr || colmax == nullptr) return LRQ_ERR_NULL;
  if (rows < 0 || hidden <= 0 || ldx < hidden || (hidden % 2) != 0) return LRQ_ERR_SHAPE;
  if ((ldx % 2) != 0 || !aligned(x, 4) || !aligned(colmax, 4)) return LRQ_ERR_ALIGN;
  hipStream_t s = (hipStream_t)stream;
  hipLaunchKernelGGL(k_zero_u32, dim3((unsigned)((hidden + 255) / 256)), dim3(256), 0, s,
                     (unsigned int*)colmax, hidden);
  int st = launch_status();
  if (st || rows == 0) return st;
  dim3 grid((unsigned)((hidden / 2 + 255) / 256), (unsigned)((rows + 63) / 64));
  hipLaunchKernelGGL(k_colmax, grid, dim3(256), 0, s, (const uint16_t*)x, ldx, rows, hidden,
                     (unsigned int*)colmax);
  return launch_status();
}

extern "C" int lrq_topk(const float* colmax, int64_t hidden, int32_t k, int32_t* idx, void* stream) {
  if (colmax == nullptr || idx == nullptr) return LRQ_ERR_NULL;
  if (hidden <= 0 || k < 0 || k > hidden || k > 1024) return LRQ_ERR_SHAPE;
  // LDS: hidden + 1024 floats, 1024 + k ints; keep within 160 KiB.
  const size_t shm = (size_t)hidden * 4 + 1024 * 4 + 1024 * 4 + (size_t)k * 4;
  if (shm > 160 * 1024) return LRQ_ERR_SHAPE;
  if (k == 0) return LRQ_OK;
  hipLaunchKernelGGL(k_topk, dim3(1), dim3(1024), shm, (hipStream_t)stream, colmax, (int)hidden, (int)k, idx);
  return launch_status();
}

extern "C" const char* lrq_status_string(int status) {
  switch (status) {
    case LRQ_OK: return "ok";
    case LRQ_ERR_NULL: return "a required pointer is NULL";
    case LRQ_ERR_SHAPE: return "invalid dimension or leading dimension";
    case LRQ_ERR_UNSUPPORTED: return "unsupported bits/group/rank/flag combination";
    case LRQ_ERR_ALIGN: return "misaligned pointer or leading dimension";
    case LRQ_ERR_WORKSPACE: return "workspace too small";
    default: return status > 0 ? hipGetErrorString((hipError_t)status) : "unknown status";
  }
}

extern "C" int32_t lrq_abi_version(void) { return 1; }
