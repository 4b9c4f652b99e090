// Residual + per-group quantisation of one unit (see lrq_common.h for the layout), shared
// by the persistent single-pass encode and the streaming second-pass / rank-0 encode.
#pragma once

#include "lrq_common.h"

namespace lrq {

// r = fp32(x - L V^T) over the lane's G/4 columns of one unit-plane, rounded once (an MFMA
// whose accumulator input is x; lopn holds -L), or r = x at rank 0.
//
// Rank 16: x reaches fp32 through the MFMA pipe instead of VALU unpacking: an identity step
// I * x (exact: one product of 1 per output, the rest zero) puts x[row][16g + 4q + v] in the
// accumulator layout, and the reconstruction step adds -L V^T to it with one rounding, as above.
template <int G, int R>
__device__ __forceinline__ void residual_plane(const u32x4 (&x)[G / 32],
                                               const u32x2 (&vop)[G / 16][R > 0 ? R / 16 : 1],
                                               const u32x2* lopn, float* r) {
  if constexpr (R == 16) {
    const int l = __lane_id();
    const u32x2 ida = identity_bop(l & 15, l >> 4);  // A operand: I[i][4g + e], e < 4, for lane (i, g)
#pragma unroll
    for (int q = 0; q < G / 16; ++q) {
      // B operand: lane (row, g) holds x[row][16g + 4q + e], e < 4 (dwords 2(q%2), +1 of x[q/2])
      const u32x2 xb = u32x2{x[q >> 1][2 * (q & 1)], x[q >> 1][2 * (q & 1) + 1]};
      f32x4 acc = mfma_16x16x16(ida, xb, zero4());
      acc = mfma_16x16x16(vop[q][0], lopn[0], acc);
      r[4 * q + 0] = acc[0];
      r[4 * q + 1] = acc[1];
      r[4 * q + 2] = acc[2];
      r[4 * q + 3] = acc[3];
    }
  } else {
#pragma unroll
    for (int k = 0; k < G / 32; ++k) unpack8(x[k], r + 8 * k);
    if constexpr (R > 0) residual_unit<G, R>(vop, lopn, r, r);
  }
}

// Lane-local min / max of n values: min(min(acc, a), b) chains, one v_min3 / v_max3 per
// two elements.
template <int n>
__device__ __forceinline__ void local_minmax(const float* r, float& mn, float& mx) {
  mn = fminf(r[0], r[1]);
  mx = fmaxf(r[0], r[1]);
#pragma unroll
  for (int e = 2; e + 1 < n; e += 2) {
    mn = fminf(fminf(mn, r[e]), r[e + 1]);
    mx = fmaxf(fmaxf(mx, r[e]), r[e + 1]);
  }
  if constexpr (n % 2 == 1) {
    mn = fminf(mn, r[n - 1]);
    mx = fmaxf(mx, r[n - 1]);
  }
}

// Quantise one unit: x[p][k] are the lane's G/4 columns of plane p (bf16); vop[p] the
// reconstruction operands of the unit-plane (unused when R == 0); lopn the NEGATED L
// operands of the lane's row; colmask an optional LDS bitmap of outlier columns (zeroed
// before the statistics).  Writes the lane's G/4 code bytes and the unit's NP (scale, zero)
// pairs.
//
// With two planes the group statistics are reduce-scattered over the row's four lanes
// (lanes 0..31 finish plane 0, lanes 32..63 plane 1), so the parameter arithmetic runs once
// for both groups, and each lane stores the pair it computed.
//
// Callers point lanes of rows past the end at the last row, with that row's inputs: their
// stores repeat its bytes, so no store is predicated (on gfx9 a predicated store makes the
// compiler drain all outstanding memory operations, prefetches included, at the next use
// of a load).
// Memory operations (stores) one call of quant_unit_core / quant_unit issues per lane: kernels
// that wait with counted vmcnt derive their counts from these.
template <int G>
constexpr int quant_core_stores() { return G / 4 / 16; }
template <int G>
constexpr int quant_unit_stores() { return quant_core_stores<G>() + 1; }

// Core of quant_unit: stores the lane's code bytes and returns the (scale, zero) pair this lane
// computed (with two planes: plane 0's in lanes 0..31, plane 1's in lanes 32..63).
template <int BITS, int G, int R>
__device__ __forceinline__ uint32_t quant_unit_core(const u32x4 (&x)[8 / BITS][G / 32],
                                                    const u32x2 (&vop)[8 / BITS][G / 16][R > 0 ? R / 16 : 1],
                                                    const u32x2* lopn, const uint32_t* colmask, int u, int N,
                                                    int g, uint8_t* __restrict__ crow) {
  constexpr int NP = 8 / BITS, E = G / 4;
  static_assert(NP == 1 || NP == 2, "group mode packs 4- or 8-bit codes");
  static_assert(E % 16 == 0 && E / 16 == quant_core_stores<G>(), "one 16-byte code store per 16 code bytes");
  float r[NP][E];
  float mn[NP], mx[NP];
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    residual_plane<G, R>(x[p], vop[p], lopn, r[p]);
    if (colmask != nullptr) {
      const int c0 = unit_base(p, u, N, NP, G) + E * g;  // E consecutive columns in one mask word
      const uint32_t mbits = colmask[c0 >> 5] >> (c0 & 31);
#pragma unroll
      for (int e = 0; e < E; ++e)
        if ((mbits >> e) & 1u) r[p][e] = 0.f;
    }
    local_minmax<E>(r[p], mn[p], mx[p]);
  }

  GroupParams gp[NP];
  uint32_t qp;
  if constexpr (NP == 2) {
    // lanes 0..31 hold plane 0's statistics, lanes 32..63 plane 1's
    const GroupParams own = group_params<BITS>(row_min4_pair(mn[0], mn[1]), row_max4_pair(mx[0], mx[1]));
    halves_broadcast(own.a, gp[0].a, gp[1].a);
    halves_broadcast(own.b, gp[0].b, gp[1].b);
    qp = own.qp;
  } else {
    gp[0] = group_params<BITS>(row_min4(mn[0]), row_max4(mx[0]));
    qp = gp[0].qp;
  }

  // byte[e]: the packed code byte of element e in bits 0..7 (higher bits are don't-care).
  // Bits BITS..7 of a code's bit pattern are zero, so plane 1's code shifted by 4 can be
  // or-ed onto plane 0's without masking.
  uint32_t byte[E];
#pragma unroll
  for (int e = 0; e < E; ++e) {
    byte[e] = quant_code_bits<BITS>(r[0][e], gp[0]);
    if constexpr (NP == 2) byte[e] = (quant_code_bits<BITS>(r[1][e], gp[1]) << 4) | byte[e];
  }
  uint32_t word[E / 4];
#pragma unroll
  for (int i = 0; i < E / 4; ++i) word[i] = gather_bytes(byte[4 * i], byte[4 * i + 1], byte[4 * i + 2], byte[4 * i + 3]);
#pragma unroll
  for (int i = 0; i < quant_core_stores<G>(); ++i)
    st16(crow + u * G + E * g + 16 * i, u32x4{word[4 * i], word[4 * i + 1], word[4 * i + 2], word[4 * i + 3]});
  return qp;
}

template <int BITS, int G, int R>
__device__ __forceinline__ void quant_unit(const u32x4 (&x)[8 / BITS][G / 32],
                                           const u32x2 (&vop)[8 / BITS][G / 16][R > 0 ? R / 16 : 1],
                                           const u32x2* lopn, const uint32_t* colmask, int u, int N, int g,
                                           uint8_t* __restrict__ crow, uint16_t* __restrict__ qrow) {
  const uint32_t qp = quant_unit_core<BITS, G, R>(x, vop, lopn, colmask, u, N, g, crow);
  static_assert(quant_unit_stores<G>() == quant_core_stores<G>() + 1, "the core's stores and one qparams store");
  if constexpr (8 / BITS == 2)
    st4(qrow + u * 4 + (g >> 1) * 2, qp);  // lanes g, g^1 write the same pair
  else
    st4(qrow + u * 2, qp);
}

// quant_unit without the qparams store: the caller gathers the pairs of several units.
template <int BITS, int G, int R>
__device__ __forceinline__ uint32_t quant_unit_regs(const u32x4 (&x)[8 / BITS][G / 32],
                                                    const u32x2 (&vop)[8 / BITS][G / 16][R > 0 ? R / 16 : 1],
                                                    const u32x2* lopn, int u, int g, uint8_t* __restrict__ crow) {
  return quant_unit_core<BITS, G, R>(x, vop, lopn, nullptr, u, 0, g, crow);
}

}  // namespace lrq
