// Small helpers on the path: bf16 transpose (basis layouts), column abs-max and top-k
// channel selection for the outlier-channel split, status strings.
#include "lrq_common.h"
#include "lrq_host.h"

#include <algorithm>

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
// Grid: (ceil(cols / 512), row groups of rows_per rows); PH waves = PH row phases x 64 column
// lanes of 8 adjacent columns (one 16-byte load per row: a wave reads 1 KB of a row), 16 loads
// in flight per thread.  The PH phases meet in LDS, so each workgroup issues one atomic per
// column (few row groups keep the atomics per address low).
template <int PH>
__global__ __launch_bounds__(PH * 64) void k_colmax(const uint16_t* __restrict__ x, int64_t ldx, int64_t rows,
                                                     int64_t cols, int64_t rows_per, unsigned int* __restrict__ colmax) {
  __shared__ float red[PH - 1][64][8];
  // the row phase is wave-uniform (readfirstlane), so the batch loop's branches are scalar: a
  // load under a per-lane branch would make the compiler wait for it at the join, and nothing
  // would overlap.  Lanes past the last column read the last 8 columns and store nothing.
  const int cl = threadIdx.x & 63, ph = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t c = ((int64_t)blockIdx.x * 64 + cl) * 8;
  const bool live = c < cols;
  const int64_t r0 = (int64_t)blockIdx.y * rows_per;
  const int64_t r1 = r0 + rows_per < rows ? r0 + rows_per : rows;
  float m[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) m[e] = 0.f;
  {
    const uint16_t* p = x + (live ? c : cols - 8);
    int64_t r = r0 + ph;
    // batches of kB rows (r, r+PH, ..., r+PH(kB-1)), the next batch in flight while one is reduced
    constexpr int kB = 16;
    u32x4 v[kB];
    auto issue = [&](int64_t rr) {
#pragma unroll
      for (int i = 0; i < kB; ++i) v[i] = ld16_stream(p + (rr + PH * i) * ldx);
    };
    auto reduce = [&](const u32x4 (&b)[kB]) {
#pragma unroll
      for (int i = 0; i < kB; ++i) {
        float f[8];
        unpack8(b[i], f);
#pragma unroll
        for (int e = 0; e < 8; ++e) m[e] = fmaxf(m[e], fabsf(f[e]));
      }
    };
    // full batches (r + PH(kB-1) < r1); the loop issues the next batch unconditionally, so the
    // wait for a batch leaves the next one in flight (a conditional issue would make the
    // compiler wait for both at the join)
    constexpr int kSpan = PH * kB;
    const int nbat =
        __builtin_amdgcn_readfirstlane(r + kSpan - PH < r1 ? (int)((r1 - r - kSpan + PH - 1) / kSpan) + 1 : 0);
    if (nbat > 0) {
      issue(r);
      for (int bi = 0; bi + 1 < nbat; ++bi) {
        u32x4 cur[kB];
#pragma unroll
        for (int i = 0; i < kB; ++i) cur[i] = v[i];
        r += kSpan;
        issue(r);
        reduce(cur);
      }
      reduce(v);
      r += kSpan;
    }
    for (; r < r1; r += PH) {
      float f[8];
      unpack8(ld16_stream(p + r * ldx), f);
#pragma unroll
      for (int e = 0; e < 8; ++e) m[e] = fmaxf(m[e], fabsf(f[e]));
    }
  }
  if (ph > 0) {
#pragma unroll
    for (int e = 0; e < 8; ++e) red[ph - 1][cl][e] = m[e];
  }
  __syncthreads();
  if (ph == 0 && live) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float a = m[e];
#pragma unroll
      for (int q = 0; q < PH - 1; ++q) a = fmaxf(a, red[q][cl][e]);
      atomicMax(colmax + c + e, __float_as_uint(a));
    }
  }
}

// Same with 2 columns per thread (4-byte loads), for rows that are not 16-byte aligned.
__global__ __launch_bounds__(256) void k_colmax2(const uint16_t* __restrict__ x, int64_t ldx, int64_t rows,
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

// Exclusive prefix sum over the 1024 threads of the workgroup (every thread calls it); also
// returns the total.  wsum: 16 words of LDS.
__device__ __forceinline__ uint32_t block_exclusive_scan(uint32_t v, uint32_t* wsum, uint32_t& total) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  uint32_t incl = v;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const uint32_t o = __shfl_up(incl, d);
    if (lane >= d) incl += o;
  }
  if (lane == 63) wsum[w] = incl;
  __syncthreads();
  uint32_t before = 0, all = 0;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const uint32_t t = wsum[i];
    before += i < w ? t : 0u;
    all += t;
  }
  __syncthreads();  // wsum may be reused by the caller's next scan
  total = all;
  return before + incl - v;
}

// Top-k by radix select in one 1024-thread workgroup.  colmax values are non-negative, so
// their fp32 bit patterns order like the values.  The k-th largest key T is fixed MSB-first,
// 8 bits per round: a 256-bin histogram of the next byte over the keys that match the bits
// fixed so far, then (wave 0) a scan from the top bin finds the bin holding the k-th key.
// The result is every column with key > T and the first k - #(key > T) columns with key == T
// (ties toward the lower index), written in ascending index order from per-thread
// contiguous chunks and two block scans.
__global__ __launch_bounds__(1024) void k_topk(const float* __restrict__ colmax, int hidden, int k,
                                               int32_t* __restrict__ idx) {
  extern __shared__ uint32_t skey[];  // hidden keys
  __shared__ uint32_t hist[256];
  __shared__ uint32_t wsum[16];
  __shared__ uint32_t s_prefix, s_need;
  const int tid = threadIdx.x, lane = tid & 63;
  for (int i = tid; i < hidden; i += 1024) skey[i] = __float_as_uint(colmax[i]);
  if (tid == 0) {
    s_prefix = 0u;
    s_need = (uint32_t)k;
  }
  uint32_t mask = 0u;
#pragma unroll 1
  for (int shift = 24; shift >= 0; shift -= 8) {
    if (tid < 256) hist[tid] = 0u;
    __syncthreads();
    const uint32_t prefix = s_prefix;
    // the keys crowd into few bins (colmax values span few exponents), so a wave adds each
    // distinct bin of its 64 keys once (ballot + popcount) instead of 64 colliding LDS atomics
    for (int it = 0; it < (hidden + 1023) / 1024; ++it) {
      const int i = it * 1024 + tid;
      const uint32_t key = i < hidden ? skey[i] : 0u;
      const uint32_t bin = (key >> shift) & 255u;
      bool pend = i < hidden && (key & mask) == prefix;
      uint64_t active = __ballot(pend);
      while (active != 0u) {
        const int leader = __ffsll((unsigned long long)active) - 1;
        const uint32_t b = __shfl(bin, leader);
        const uint64_t same = __ballot(pend && bin == b);
        if (lane == leader) atomicAdd(&hist[b], (uint32_t)__popcll(same));
        pend = pend && bin != b;
        active &= ~same;
      }
    }
    __syncthreads();
    if (tid < 64) {
      // lane l holds bins 255-4l .. 252-4l (top first)
      uint32_t cnt[4], tot = 0;
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        cnt[m] = hist[255 - (4 * lane + m)];
        tot += cnt[m];
      }
      uint32_t incl = tot;
#pragma unroll
      for (int d = 1; d < 64; d <<= 1) {
        const uint32_t o = __shfl_up(incl, d);
        if (lane >= d) incl += o;
      }
      const uint32_t need = s_need;
      uint32_t cum = incl - tot;
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        if (cum < need && cum + cnt[m] >= need) {
          s_prefix = prefix | ((uint32_t)(255 - (4 * lane + m)) << shift);
          s_need = need - cum;
        }
        cum += cnt[m];
      }
    }
    mask |= 255u << shift;
    __syncthreads();
  }
  const uint32_t T = s_prefix, need_eq = s_need;  // take the first need_eq keys equal to T
  const int C = (hidden + 1023) / 1024, i0 = tid * C, i1 = min(i0 + C, hidden);
  uint32_t n_gt = 0, n_eq = 0;
  for (int i = i0; i < i1; ++i) {
    const uint32_t key = skey[i];
    n_gt += key > T;
    n_eq += key == T;
  }
  uint32_t tot;
  const uint32_t eq_before = block_exclusive_scan(n_eq, wsum, tot);
  const uint32_t take_eq = eq_before >= need_eq ? 0u : min(n_eq, need_eq - eq_before);
  uint32_t pos = block_exclusive_scan(n_gt + take_eq, wsum, tot);
  uint32_t eq_seen = 0;
  for (int i = i0; i < i1; ++i) {
    const uint32_t key = skey[i];
    bool sel = key > T;
    if (key == T) {
      sel = eq_seen < take_eq;
      ++eq_seen;
    }
    if (sel) idx[pos++] = i;
  }
  (void)lane;
}

}  // namespace lrq

using namespace lrq;

extern "C" int lrq_transpose_bf16(const void* src, int64_t rows, int64_t cols, void* dst, void* stream) {
  if (src == nullptr || dst == nullptr) return LRQ_ERR_NULL;
  if (rows < 0 || cols < 0) return LRQ_ERR_SHAPE;
  if (!aligned(src, 2) || !aligned(dst, 2)) return LRQ_ERR_ALIGN;
  if (rows == 0 || cols == 0) return LRQ_OK;
  dim3 grid((unsigned)((cols + 31) / 32), (unsigned)((rows + 31) / 32));
  LRQ_TRY(launch(k_transpose_bf16, grid, dim3(256), 0, (hipStream_t)stream, (const uint16_t*)src, rows,
                     cols, (uint16_t*)dst));
  return LRQ_OK;
}

// k_colmax launch shape: one workgroup of 8 waves per CU (c3 shape, colmax entry: 36.1 us;
// 4 waves x 4 per CU 39.3, 8 x 2 40.0, 16 x 1 39.5, 16 x 2 37.6)
static constexpr int kColmaxPhases = 8, kColmaxWgPerCu = 1;
extern "C" int lrq_colmax(const void* x, int64_t ldx, int64_t rows, int64_t hidden, float* colmax,
                          void* stream) {
  if (x == nullptr || colmax == nullptr) return LRQ_ERR_NULL;
  if (rows < 0 || hidden <= 0 || ldx < hidden || (hidden % 2) != 0) return LRQ_ERR_SHAPE;
  if ((ldx % 2) != 0 || !aligned(x, 4) || !aligned(colmax, 4)) return LRQ_ERR_ALIGN;
  hipStream_t s = (hipStream_t)stream;
  LRQ_TRY(launch(k_zero_u32, dim3((unsigned)((hidden + 255) / 256)), dim3(256), 0, s,
                     (unsigned int*)colmax, hidden));
  if (rows == 0) return LRQ_OK;
  if ((hidden % 8) == 0 && (ldx % 8) == 0 && aligned(x, 16)) {
    // about kColmaxWgPerCu workgroups of kColmaxPhases waves per CU (one atomic per column per
    // workgroup), row groups of whole PH * 16-row steps (PH phases x 16-row batches)
    constexpr int PH = kColmaxPhases;
    const int64_t cgroups = (hidden + 511) / 512;
    int64_t groups = std::max<int64_t>(1, (int64_t)cu_count() * kColmaxWgPerCu / cgroups);
    int64_t rows_per = (rows + groups - 1) / groups;
    rows_per = (rows_per + 16 * PH - 1) / (16 * PH) * (16 * PH);
    groups = (rows + rows_per - 1) / rows_per;
    LRQ_TRY(launch(k_colmax<PH>, dim3((unsigned)cgroups, (unsigned)groups), dim3(PH * 64), 0, s, (const uint16_t*)x,
                   ldx, rows, hidden, rows_per, (unsigned int*)colmax));
  } else {
    dim3 grid((unsigned)((hidden / 2 + 255) / 256), (unsigned)((rows + 63) / 64));
    LRQ_TRY(launch(k_colmax2, grid, dim3(256), 0, s, (const uint16_t*)x, ldx, rows, hidden,
                       (unsigned int*)colmax));
  }
  return LRQ_OK;
}

extern "C" int lrq_topk(const float* colmax, int64_t hidden, int32_t k, int32_t* idx, void* stream) {
  if (colmax == nullptr || idx == nullptr) return LRQ_ERR_NULL;
  if (hidden <= 0 || k < 0 || k > hidden) return LRQ_ERR_SHAPE;
  // LDS: the hidden keys plus about 1.1 KiB of static histogram and scan words; 160 KiB total.
  const size_t shm = (size_t)hidden * 4;
  if (shm + 2048 > 160 * 1024) return LRQ_ERR_SHAPE;
  if (k == 0) return LRQ_OK;
  LRQ_TRY(launch(k_topk, dim3(1), dim3(1024), shm, (hipStream_t)stream, colmax, (int)hidden, (int)k, idx));
  return LRQ_OK;
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
