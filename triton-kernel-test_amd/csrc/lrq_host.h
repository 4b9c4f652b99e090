// Host-side argument validation shared by the C-ABI entry points.  Every check here runs
// before any HIP call, so an invalid argument returns a negative status without touching
// the GPU (the CPU test-suite drives these paths with no device present).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>
#include <cstring>
#include <initializer_list>
#include <tuple>
#include <type_traits>
#include <utility>

#include "../../include/lrq.h"

namespace lrq {

static inline bool aligned(const void* p, uintptr_t a) { return ((uintptr_t)p % a) == 0; }

// fp32 -> bf16 (round to nearest even) on the host, and back.
static inline uint16_t bf16_bits_host(float f) {
  uint32_t u;
  std::memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);  // quiet NaN
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}
static inline float bf16_value_host(uint16_t h) {
  const uint32_t u = (uint32_t)h << 16;
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}

static constexpr int format_key(int bits, int group, int rank) { return bits * 100000 + group * 100 + rank; }

// Compute units of the current device (256 on MI355X); launch shapes are sized from it.  The
// attribute is read once per device and kept (a constant of the hardware, so the cache is
// the same for every caller and thread; a racing first read stores the same value).
static inline int cu_count() {
  constexpr int kMaxDev = 64;
  static std::atomic<int> cached[kMaxDev];
  int dev = 0, n = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 256;
  if (dev >= 0 && dev < kMaxDev) {
    const int c = cached[dev].load(std::memory_order_relaxed);
    if (c > 0) return c;
  }
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) return 256;
  if (dev >= 0 && dev < kMaxDev) cached[dev].store(n, std::memory_order_relaxed);
  return n;
}

// Launches kernel k and returns the status of this launch only: hipLaunchKernel's own
// result, so an error that an earlier call left on the thread is neither reported here nor
// cleared.  The arguments are converted to the kernel's parameter types first.
template <typename... P, typename... A>
static inline int launch(void (*k)(P...), dim3 grid, dim3 block, size_t shm, hipStream_t s, A&&... args) {
  static_assert(sizeof...(P) == sizeof...(A), "kernel argument count");
  std::tuple<std::decay_t<P>...> params(std::forward<A>(args)...);
  void* argv[sizeof...(P) > 0 ? sizeof...(P) : 1];
  std::apply([&](auto&... p) {
    int i = 0;
    ((argv[i++] = (void*)&p), ...);
  }, params);
  const hipError_t e = hipLaunchKernel((const void*)k, grid, block, argv, shm, s);
  return e == hipSuccess ? LRQ_OK : (int)e;
}

// Returns from the enclosing function with a non-zero status.
#define LRQ_TRY(expr)                            \
  do {                                           \
    const int lrq_try_status_ = (expr);          \
    if (lrq_try_status_ != LRQ_OK) return lrq_try_status_; \
  } while (0)

// Validates a group-mode descriptor (Vt is checked by the two-pass encode, its only reader).
static inline int validate_tensors(const lrq_tensors* t) {
  if (t == nullptr) return LRQ_ERR_NULL;
  if (t->rows < 0 || t->hidden <= 0 || t->rows > INT32_MAX || t->hidden > INT32_MAX) return LRQ_ERR_SHAPE;
  if (t->bits != 4 && t->bits != 8) return LRQ_ERR_UNSUPPORTED;
  if (t->group != 64 && t->group != 128) return LRQ_ERR_UNSUPPORTED;
  if (t->rank != 0 && t->rank != 16 && t->rank != 32) return LRQ_ERR_UNSUPPORTED;
  if ((t->flags & ~LRQ_FLAG_HADAMARD) != 0) return LRQ_ERR_UNSUPPORTED;
  const int64_t np = 8 / t->bits;
  if (t->hidden % (t->group * np) != 0) return LRQ_ERR_SHAPE;
  if ((t->flags & LRQ_FLAG_HADAMARD) && t->hidden % 128 != 0) return LRQ_ERR_SHAPE;
  if (t->rank > 0) {
    if (t->L == nullptr || t->V == nullptr) return LRQ_ERR_NULL;
    if (t->ld_L < t->rank) return LRQ_ERR_SHAPE;
    if ((t->ld_L % 4) != 0 || !aligned(t->L, 8) || !aligned(t->V, 8)) return LRQ_ERR_ALIGN;
    if (t->Vt != nullptr && !aligned(t->Vt, 16)) return LRQ_ERR_ALIGN;
  }
  if (t->codes == nullptr || t->qparams == nullptr) return LRQ_ERR_NULL;
  if (t->ld_codes < t->hidden * t->bits / 8 || t->ld_qp < 2 * (t->hidden / t->group)) return LRQ_ERR_SHAPE;
  if ((t->ld_codes % 16) != 0 || !aligned(t->codes, 16)) return LRQ_ERR_ALIGN;
  if ((t->ld_qp % 4) != 0 || !aligned(t->qparams, 8)) return LRQ_ERR_ALIGN;
  if (t->n_outlier < 0 || t->n_outlier > t->hidden) return LRQ_ERR_SHAPE;
  if (t->n_outlier > 0) {
    if (t->outlier_idx == nullptr || t->side == nullptr) return LRQ_ERR_NULL;
    if (t->ld_side < t->n_outlier) return LRQ_ERR_SHAPE;
    if (!aligned(t->side, 2) || !aligned(t->outlier_idx, 4)) return LRQ_ERR_ALIGN;
  }
  return LRQ_OK;
}

// A bf16 [rows, >= cols] operand with 16-byte aligned rows.
static inline int validate_rows16(const void* p, int64_t ld, int64_t cols) {
  if (p == nullptr) return LRQ_ERR_NULL;
  if (ld < cols) return LRQ_ERR_SHAPE;
  if ((ld % 8) != 0 || !aligned(p, 16)) return LRQ_ERR_ALIGN;
  return LRQ_OK;
}

}  // namespace lrq
