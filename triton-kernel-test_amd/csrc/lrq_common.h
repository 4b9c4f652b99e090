// Shared device helpers for the compressed-activation kernels (gfx950 / CDNA4, wave64).
//
// Layout conventions used by every group-mode kernel in this library.
//
//  * A wave works on a block of 16 rows.  Lane l has j = l & 15 (row inside the block)
//    and g = l >> 4 (0..3).
//  * Columns are split into NP = 8/bits packing planes (plane p holds columns
//    [p*N/NP, (p+1)*N/NP)); byte c of a packed code row holds column c of every plane.
//  * A "unit" u is group-column u of every plane: columns base_p = p*N/NP + u*G .. +G-1.
//    Lane (j, g) owns the G/4 consecutive columns base_p + (G/4)*g + e, e < G/4, of row j,
//    for every plane; they sit in G/32 16-byte vectors x[p][k] (columns 8k .. 8k+7 of the
//    lane's quarter, two bf16 per dword, even column low).  The lane's codes for the unit
//    are the G/4 contiguous bytes u*G + (G/4)*g .. of the packed row.
//  * Reconstruction L V^T: v_mfma_f32_16x16x16_bf16 number q (q < G/16) of a unit-plane
//    feeds A row i with V row base_p + (G/4)*(i/4) + 4q + (i%4) (ranks 4g..4g+3 of the
//    rank tile in lane (i, g)) and B = L^T; its output lands in lane (j, g) as columns
//    base_p + (G/4)*g + 4q + v, v < 4 — exactly elements 4q..4q+3 of the lane's quarter.
//  * Projection L = Y V: the same operand, multiplied by the identity on MFMA, comes out
//    transposed (lane (rank, g) holding V at columns base_p + (G/4)g + 4q + v), which is
//    the A operand of a 16x16x16 MFMA whose B operand is the lane's own x elements
//    4q..4q+3.  Its output is L[row j][16t + 4g + v] in lane (j, g): the B operand the
//    reconstruction needs.  No activation data ever moves between lanes.
//  * Group statistics: the four lanes of a row (j, j+16, j+32, j+48) hold the whole group;
//    two permlane swaps finish min/max.  With two planes the two groups of a unit are
//    reduce-scattered (lanes 0..31 finish plane 0, 32..63 plane 1), their parameters are
//    computed once and swapped back.
//  * qparams: fp16 [rows, N/(G*NP), NP, 2] — per unit, (scale, zero) of each plane's group.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

#include <type_traits>

namespace lrq {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

static constexpr int kWave = 64;

// ---------------------------------------------------------------- bf16 / fp16
__device__ __forceinline__ float bf_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// fp32 -> 2 x bf16 in one dword (lo in bits 0..15), round to nearest even, on the gfx950
// conversion unit (v_cvt_pk_bf16_f32).
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t){lo, hi}, bf16x2_t));
}
__device__ __forceinline__ float bf16_roundtrip(float f) { return __uint_as_float(pack_bf16x2(f, 0.f) << 16); }
// bf16_roundtrip of two values with one conversion.
__device__ __forceinline__ void bf16_roundtrip2(float& a, float& b) {
  const uint32_t w = pack_bf16x2(a, b);
  a = __uint_as_float(w << 16);
  b = __uint_as_float(w & 0xffff0000u);
}
// Pack two fp32 values that are already exactly representable in bf16 (no rounding): the
// high halves of both, one v_perm_b32.
__device__ __forceinline__ uint32_t pack_bf16x2_exact(float lo, float hi) {
  return __builtin_amdgcn_perm(__float_as_uint(hi), __float_as_uint(lo), 0x07060302u);
}

// Byte K of w as fp32 (v_cvt_f32_ubyteK).  Written as asm so the compiler keeps one
// masked dword feeding four conversions instead of splitting it into per-byte extracts.
template <int K>
__device__ __forceinline__ float ubyte_f32(uint32_t w) {
  float f;
  if constexpr (K == 0) asm("v_cvt_f32_ubyte0 %0, %1" : "=v"(f) : "v"(w));
  else if constexpr (K == 1) asm("v_cvt_f32_ubyte1 %0, %1" : "=v"(f) : "v"(w));
  else if constexpr (K == 2) asm("v_cvt_f32_ubyte2 %0, %1" : "=v"(f) : "v"(w));
  else asm("v_cvt_f32_ubyte3 %0, %1" : "=v"(f) : "v"(w));
  return f;
}

// fp32 -> fp16 bits (RNE) and back.
__device__ __forceinline__ uint16_t f16_bits(float f) {
  return __builtin_bit_cast(uint16_t, (_Float16)f);
}
__device__ __forceinline__ float f16_val(uint32_t h) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}

// ---------------------------------------------------------------- MFMA wrappers
// D(16x16) += A(16x32) * B(32x16), bf16 inputs, fp32 accumulate.
__device__ __forceinline__ f32x4 mfma_16x16x32(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                 __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}
// D(16x16) += A(16x16) * B(16x16), bf16 inputs, fp32 accumulate.
__device__ __forceinline__ f32x4 mfma_16x16x16(u32x2 a, u32x2 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s16x4, a),
                                                   __builtin_bit_cast(s16x4, b), c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 zero4() { return f32x4{0.f, 0.f, 0.f, 0.f}; }

// ---------------------------------------------------------------- memory helpers
__device__ __forceinline__ u32x4 ld16(const void* p) { return *reinterpret_cast<const u32x4*>(p); }
__device__ __forceinline__ u32x2 ld8(const void* p) { return *reinterpret_cast<const u32x2*>(p); }
__device__ __forceinline__ uint32_t ld4(const void* p) { return *reinterpret_cast<const uint32_t*>(p); }
__device__ __forceinline__ u32x4 ld16_stream(const void* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}
__device__ __forceinline__ u32x2 ld8_stream(const void* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(p));
}
// s_waitcnt immediate for vmcnt(n), n < 64 (gfx9: low bits [3:0], high bits [15:14]); expcnt
// and lgkmcnt are not waited for.
constexpr int vmcnt_imm(int n) { return 0x0f70 | (n & 15) | ((n >> 4) << 14); }

// f(std::integral_constant<int, i>) for i = I .. N-1, unrolled at compile time (each call sees
// its index as a constant expression, e.g. for a counted wait).
template <int I, int N, class F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>{});
    static_for<I + 1, N>(f);
  }
}

// Make a register value opaque to the compiler: it can no longer be recomputed or reloaded
// from memory at a later use, so operands loaded once for a whole loop stay in registers.
__device__ __forceinline__ void pin(u32x2& v) { asm volatile("" : "+v"(v)); }
__device__ __forceinline__ void pin(u32x4& v) { asm volatile("" : "+v"(v)); }
__device__ __forceinline__ void st16(void* p, u32x4 v) { *reinterpret_cast<u32x4*>(p) = v; }
__device__ __forceinline__ void st8(void* p, u32x2 v) { *reinterpret_cast<u32x2*>(p) = v; }
__device__ __forceinline__ void st4(void* p, uint32_t v) { *reinterpret_cast<uint32_t*>(p) = v; }
__device__ __forceinline__ void st16_stream(void* p, u32x4 v) {
  __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(p));
}

// A pointer the caller knows to be wave-uniform, in scalar registers: a buffer resource built from
// a base the compiler cannot prove uniform is wrapped in a waterfall loop (one pass per distinct
// value, with compares and exec-mask updates around every buffer access).
template <class T>
__device__ __forceinline__ T* uniform_ptr(T* p) {
  const uint64_t v = reinterpret_cast<uint64_t>(p);
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return reinterpret_cast<T*>(((uint64_t)hi << 32) | lo);
}

// XCD-aware tile order: workgroup i of an n-workgroup launch runs on XCD i % 8 (round-robin
// dispatch).  The returned tile index gives each XCD one contiguous range of tiles, walked in
// order, so workgroups that run together on one XCD (one L2) take neighbouring tiles.  A bijection
// of [0, n).
__device__ __forceinline__ int xcd_tile(int i, int n) {
  const int per = n / 8, rem = n % 8, x = i % 8, k = i / 8;
  return x < rem ? x * (per + 1) + k : rem * (per + 1) + (x - rem) * per + k;
}

// Raw buffer resource over the `len`-byte region at `base`, both wave-uniform by the caller's
// contract; they are moved to scalar registers so the compiler emits no waterfall loop.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t uniform_rsrc(void* base, uint32_t len) {
  return __builtin_amdgcn_make_buffer_rsrc(uniform_ptr(base), (short)0,
                                           (int)__builtin_amdgcn_readfirstlane(len), 0x00020000);
}

// Predicated 8-byte store without a branch: a raw buffer store over the `len`-byte region at
// the wave-uniform `base`; lanes with !keep use an offset past the region, which the
// hardware drops.  (A branch around a store would make the compiler drain every
// outstanding memory operation at the next use of a load — gfx9 counts loads and stores
// in one in-order counter.)
__device__ __forceinline__ void st8_pred(void* base, uint32_t len, uint32_t off, u32x2 v, bool keep) {
  const __amdgpu_buffer_rsrc_t r = uniform_rsrc(base, len);
  __builtin_amdgcn_raw_buffer_store_b64(v, r, keep ? off : 0x7ffffff0u, 0, 0);
}

// 16-byte form of st8_pred (offset 16-byte aligned within the region).
__device__ __forceinline__ void st16_pred(void* base, uint32_t len, uint32_t off, u32x4 v, bool keep) {
  const __amdgpu_buffer_rsrc_t r = uniform_rsrc(base, len);
  __builtin_amdgcn_raw_buffer_store_b128(v, r, keep ? off : 0x7ffffff0u, 0, 0);
}
// st16_pred as a non-temporal (streaming) store.
__device__ __forceinline__ void st16_pred_stream(void* base, uint32_t len, uint32_t off, u32x4 v, bool keep) {
  const __amdgpu_buffer_rsrc_t r = uniform_rsrc(base, len);
  __builtin_amdgcn_raw_buffer_store_b128(v, r, keep ? off : 0x7ffffff0u, 0, 2);
}

// Unpack the 8 bf16 of a 16-byte vector into fp32.
__device__ __forceinline__ void unpack8(u32x4 v, float* f) {
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    f[2 * d] = bf_lo(v[d]);
    f[2 * d + 1] = bf_hi(v[d]);
  }
}
__device__ __forceinline__ u32x4 pack8(const float* f) {
  u32x4 v;
#pragma unroll
  for (int d = 0; d < 4; ++d) v[d] = pack_bf16x2(f[2 * d], f[2 * d + 1]);
  return v;
}

// ---------------------------------------------------------------- unit geometry
// First column of unit u in plane p.
__device__ __forceinline__ int unit_base(int p, int u, int N, int NP, int G) { return p * (N / NP) + u * G; }

// V row feeding A row j of reconstruction MFMA q (see the header comment).
template <int G>
__device__ __forceinline__ int vrow_res(int base, int j, int q) {
  return base + (G / 4) * (j >> 2) + 4 * q + (j & 3);
}

// Load the reconstruction A operands of one unit-plane: vop[q][t] for q < G/16, t < R/16.
template <int G, int R>
__device__ __forceinline__ void load_vops(const uint16_t* __restrict__ V, int base, int j, int g,
                                          u32x2 (&vop)[G / 16][R / 16]) {
#pragma unroll
  for (int q = 0; q < G / 16; ++q)
#pragma unroll
    for (int t = 0; t < R / 16; ++t)
      vop[q][t] = ld8(V + (int64_t)vrow_res<G>(base, j, q) * R + 16 * t + 4 * g);
}

// out[4q + v] = fp32(c[4q + v] + sum_rank V[col][rank] * L[row][rank]) for the lane's G/4
// columns of one unit-plane, rounded once: the MFMA adds its C operand and all products
// exactly before rounding (checked on gfx950).  Rank 16 is one 16x16x16 step; rank 32 is one
// 16x16x32 step whose K order puts ranks 4g..4g+3 and 16+4g..16+4g+3 in lane group g, so
// the two 16-rank operands are simply concatenated.  Pass L negated to subtract.
template <int G, int R>
__device__ __forceinline__ void residual_unit(const u32x2 (&vop)[G / 16][R / 16], const u32x2* lop,
                                              const float* c, float* out) {
  static_assert(R == 16 || R == 32, "rank 16 or 32");
#pragma unroll
  for (int q = 0; q < G / 16; ++q) {
    f32x4 acc = f32x4{c[4 * q], c[4 * q + 1], c[4 * q + 2], c[4 * q + 3]};
    if constexpr (R == 16) {
      acc = mfma_16x16x16(vop[q][0], lop[0], acc);
    } else {
      const u32x4 a = u32x4{vop[q][0][0], vop[q][0][1], vop[q][1][0], vop[q][1][1]};
      const u32x4 b = u32x4{lop[0][0], lop[0][1], lop[1][0], lop[1][1]};
      acc = mfma_16x16x32(a, b, acc);
    }
    out[4 * q + 0] = acc[0];
    out[4 * q + 1] = acc[1];
    out[4 * q + 2] = acc[2];
    out[4 * q + 3] = acc[3];
  }
}

// Negate packed bf16 operands (exact).
__device__ __forceinline__ u32x2 neg_bf16x4(u32x2 v) { return u32x2{v[0] ^ 0x80008000u, v[1] ^ 0x80008000u}; }

// B operand of the identity: lane (j, g) holds I[4g + e][j], e < 4, as bf16.
__device__ __forceinline__ u32x2 identity_bop(int j, int g) {
  const uint32_t one = 0x3f80u;
  uint32_t h[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) h[e] = (4 * g + e == j) ? one : 0u;
  return u32x2{h[0] | (h[1] << 16), h[2] | (h[3] << 16)};
}

// Projection partial for one unit-plane: acc[t] += V_t^T(cols) * X^T(cols) over the lane
// quarter's G/4 columns.  The V^T operand comes from multiplying the reconstruction operand
// by the identity (exact): operands q and q+1 transpose to lane (rank, g) holding V at the
// 8 consecutive columns 8*(q/2) .. +7 of quarter g, which pair with x[q/2] as a 16x16x32 step.
template <int G, int R>
__device__ __forceinline__ void project_unit(const u32x2 (&vop)[G / 16][R / 16], const u32x4* x, u32x2 ident,
                                             f32x4* acc) {
#pragma unroll
  for (int k = 0; k < G / 32; ++k) {
#pragma unroll
    for (int t = 0; t < R / 16; ++t) {
      const f32x4 v0 = mfma_16x16x16(vop[2 * k][t], ident, zero4());
      const f32x4 v1 = mfma_16x16x16(vop[2 * k + 1][t], ident, zero4());
      const u32x4 a = u32x4{pack_bf16x2_exact(v0[0], v0[1]), pack_bf16x2_exact(v0[2], v0[3]),
                            pack_bf16x2_exact(v1[0], v1[1]), pack_bf16x2_exact(v1[2], v1[3])};
      acc[t] = mfma_16x16x32(a, x[k], acc[t]);
    }
  }
}

// The V^T operands of project_unit, computed once: vt[k][t] is the A operand that pairs with
// x[k] (see project_unit) for rank tile t.
template <int G, int R>
__device__ __forceinline__ void transpose_vops(const u32x2 (&vop)[G / 16][R / 16], u32x2 ident,
                                               u32x4 (&vt)[G / 32][R / 16]) {
#pragma unroll
  for (int k = 0; k < G / 32; ++k) {
#pragma unroll
    for (int t = 0; t < R / 16; ++t) {
      const f32x4 v0 = mfma_16x16x16(vop[2 * k][t], ident, zero4());
      const f32x4 v1 = mfma_16x16x16(vop[2 * k + 1][t], ident, zero4());
      vt[k][t] = u32x4{pack_bf16x2_exact(v0[0], v0[1]), pack_bf16x2_exact(v0[2], v0[3]),
                       pack_bf16x2_exact(v1[0], v1[1]), pack_bf16x2_exact(v1[2], v1[3])};
    }
  }
}
// project_unit with the V^T operands already transposed.
template <int G, int R>
__device__ __forceinline__ void project_unit_vt(const u32x4 (&vt)[G / 32][R / 16], const u32x4* x, f32x4* acc) {
#pragma unroll
  for (int k = 0; k < G / 32; ++k)
#pragma unroll
    for (int t = 0; t < R / 16; ++t) acc[t] = mfma_16x16x32(vt[k][t], x[k], acc[t]);
}

// 16 bytes per lane from global memory straight into LDS (no VGPRs): lane l's bytes land at
// lds + 16 * l, so `lds` must be wave-uniform.  Non-temporal (streamed once).  Completion is
// counted by vmcnt.
__device__ __forceinline__ void ld16_to_lds(const void* g, void* lds) {
  __builtin_amdgcn_global_load_lds(g, (__attribute__((address_space(3))) void*)lds, 16, 0, 2);
}

// ---------------------------------------------------------------- row-quad exchanges
// The four lanes of a row (j, j+16, j+32, j+48) are one lane of each 16-lane row of the
// wave.  v_permlane32_swap exchanges lanes 32..63 of its first operand with lanes 0..31 of
// its second; v_permlane16_swap exchanges the odd 16-lane rows of its first operand with the
// even rows of its second.  Both are plain VALU moves (no LDS round trip).
__device__ __forceinline__ void swap32(float& a, float& b) {
  const auto s = __builtin_amdgcn_permlane32_swap(__float_as_uint(a), __float_as_uint(b), false, false);
  a = __uint_as_float(s[0]);
  b = __uint_as_float(s[1]);
}
__device__ __forceinline__ void swap16(float& a, float& b) {
  const auto s = __builtin_amdgcn_permlane16_swap(__float_as_uint(a), __float_as_uint(b), false, false);
  a = __uint_as_float(s[0]);
  b = __uint_as_float(s[1]);
}
// min / max of non-NaN values without the canonicalising moves the compiler adds around
// fminf / fmaxf (and around v_med3 against an infinity, which it folds into min / max) of
// values it cannot prove canonical, such as permlane results.
__device__ __forceinline__ float min_nc(float a, float b) {
  float r;
  asm("v_min_f32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
  return r;
}
__device__ __forceinline__ float max_nc(float a, float b) {
  float r;
  asm("v_max_f32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
  return r;
}

// Reductions over the four lanes of a row; every lane receives the result.
__device__ __forceinline__ float row_min4(float v) {
  float a = v, b = v;
  swap32(a, b);  // a = v of lanes 0..31 repeated, b = v of lanes 32..63 repeated
  v = min_nc(a, b);
  a = v, b = v;
  swap16(a, b);
  return min_nc(a, b);
}
__device__ __forceinline__ float row_max4(float v) {
  float a = v, b = v;
  swap32(a, b);
  v = max_nc(a, b);
  a = v, b = v;
  swap16(a, b);
  return max_nc(a, b);
}
// Reduce-scatter of two per-lane partials over the row: lanes 0..31 receive the min of
// `va` over the row's four lanes, lanes 32..63 the min of `vb`.
__device__ __forceinline__ float row_min4_pair(float va, float vb) {
  swap32(va, vb);  // va = [a(l), b(l)], vb = [a(l+32), b(l+32)] for lanes l < 32 | l >= 32
  float v = min_nc(va, vb);
  float a = v, b = v;
  swap16(a, b);
  return min_nc(a, b);
}
__device__ __forceinline__ float row_max4_pair(float va, float vb) {
  swap32(va, vb);
  float v = max_nc(va, vb);
  float a = v, b = v;
  swap16(a, b);
  return max_nc(a, b);
}
// Exclusive prefix sum of `v` over the row's four lanes in lane-group order g = 0 .. 3 (lane
// 16g + j), and the row's total.
__device__ __forceinline__ void row_prefix4(uint32_t v, int g, uint32_t& pre, uint32_t& total) {
  const auto h = __builtin_amdgcn_permlane16_swap(v, v, false, false);  // v of groups g & ~1, g | 1
  const auto q = __builtin_amdgcn_permlane32_swap(h[0] + h[1], h[0] + h[1], false, false);
  // q[0] = the sum over groups 0 and 1, q[1] = over groups 2 and 3
  pre = ((g & 1) ? h[0] : 0u) + ((g & 2) ? q[0] : 0u);
  total = q[0] + q[1];
}
// Bitwise or of `v` over the row's four lanes.
__device__ __forceinline__ uint32_t row_or4(uint32_t v) {
  const auto h = __builtin_amdgcn_permlane16_swap(v, v, false, false);
  const auto q = __builtin_amdgcn_permlane32_swap(h[0] | h[1], h[0] | h[1], false, false);
  return q[0] | q[1];
}
// Inverse of the pair scatter: `v` holds one value in lanes 0..31 and another in 32..63;
// returns the first in lo and the second in hi, in every lane.
__device__ __forceinline__ void halves_broadcast(float v, float& lo, float& hi) {
  lo = v, hi = v;
  swap32(lo, hi);
}
__device__ __forceinline__ float wave_sum4(float v) {
  v += __shfl_xor(v, 16);
  v += __shfl_xor(v, 32);
  return v;
}

// Workgroup barrier that waits for LDS traffic only (outstanding global loads — e.g. a
// prefetch of the next row block — stay in flight across it).
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0); vmcnt, expcnt untouched
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// ---------------------------------------------------------------- group quantiser
// Per-group parameters from min/max, exactly as the CPU oracle defines them:
//   scale_h = fp16(min((mx - mn) * fp32(1/qmax), 65504)), 1 when that is 0;
//   zero_h  = fp16(clamp(mn)); inv = 1 / fp32(scale_h) correctly rounded;
//   a = fp32(inv * fp32(1/qmax)); b = fp32(-fp32(zero_h) * a).
// The reciprocal is rcp + one Newton step, which equals the correctly rounded 1/x for every
// positive finite fp16 x (checked exhaustively on gfx950).
struct GroupParams {
  float a, b;
  uint32_t qp;  // scale_h | zero_h << 16, the qparams pair as stored
};
template <int BITS>
__device__ __forceinline__ GroupParams group_params(float mn, float mx) {
  constexpr float kInvQmax = 1.0f / (float)((1 << BITS) - 1);
  GroupParams gp;
  const float s = fminf(__fmul_rn(__fsub_rn(mx, mn), kInvQmax), 65504.f);
  uint32_t sh = f16_bits(s);
  if ((sh & 0x7fffu) == 0) sh = 0x3c00u;  // 1.0
  const uint32_t zh = f16_bits(__builtin_amdgcn_fmed3f(mn, -65504.f, 65504.f));
  gp.qp = sh | (zh << 16);
  const float sf = f16_val(sh);
  const float r0 = __builtin_amdgcn_rcpf(sf);
  const float inv = __builtin_fmaf(__builtin_fmaf(-sf, r0, 1.0f), r0, r0);
  gp.a = __fmul_rn(inv, kInvQmax);
  gp.b = __fmul_rn(-f16_val(zh), gp.a);
  return gp;
}
// code = rint(qmax * clamp(fma(r, a, b), 0, 1)), returned as the bit pattern of
// 1.5*2^23 + code: the clamp folds into the fma (clamp modifier; NaN gives 0), and
// fma(u, qmax, 1.5*2^23) rounds u*qmax to an integer (half to even) in the low mantissa
// bits, so the code is the low BITS bits of the result and bits BITS..7 are zero.
template <int BITS>
__device__ __forceinline__ uint32_t quant_code_bits(float r, const GroupParams& gp) {
  constexpr float qmax = (float)((1 << BITS) - 1);
  const float u = __builtin_amdgcn_fmed3f(__builtin_fmaf(r, gp.a, gp.b), 0.f, 1.f);
  return __float_as_uint(__builtin_fmaf(u, qmax, 12582912.0f));
}
// Gather byte 0 of four dwords into one dword (b0 in bits 0..7).
__device__ __forceinline__ uint32_t gather_bytes(uint32_t b0, uint32_t b1, uint32_t b2, uint32_t b3) {
  const uint32_t lo = __builtin_amdgcn_perm(b1, b0, 0x0c0c0400u);  // [b0.0, b1.0, 0, 0]
  const uint32_t hi = __builtin_amdgcn_perm(b3, b2, 0x04000c0cu);  // [0, 0, b2.0, b3.0]
  return lo | hi;
}

}  // namespace lrq
