// Residual + per-group quantisation of one unit (see lrq_common.h for the layout), shared
// by the persistent single-pass encode and the streaming second-pass / rank-0 encode.
#pragma once

#include "lrq_common.h"

namespace lrq {

// x[p][k]: the lane's G/4 columns of plane p (bf16); vop[p]: reconstruction operands of the
// unit-plane (unused when R == 0); lop: L operands of the lane's row; colmask: optional LDS
// bitmap of outlier columns (zeroed before the statistics).  Writes the lane's G/4 code bytes
// and the unit's NP (scale, zero) pairs.  Callers point lanes of rows past the end at the
// last row, with that row's inputs: their stores repeat its bytes, so no store is predicated
// (on gfx9 a predicated store makes the compiler drain all outstanding memory operations,
// prefetches included, at the next use of a load).
template <int BITS, int G, int R>
__device__ __forceinline__ void quant_unit(const u32x4 (&x)[8 / BITS][G / 32],
                                           const u32x2 (&vop)[8 / BITS][G / 16][R > 0 ? R / 16 : 1],
                                           const u32x2* lop, const uint32_t* colmask, int u, int N, int g,
                                           uint8_t* __restrict__ crow, uint16_t* __restrict__ qrow) {
  constexpr int NP = 8 / BITS, E = G / 4;
  static_assert(NP == 1 || NP == 2, "group mode packs 4- or 8-bit codes");
  // byte[e]: the packed code byte of element e in bits 0..7 (higher bits are don't-care)
  uint32_t byte[E];
  uint32_t qp[NP];

#pragma unroll
  for (int p = 0; p < NP; ++p) {
    float r[E];
#pragma unroll
    for (int k = 0; k < G / 32; ++k) unpack8(x[p][k], r + 8 * k);
    if constexpr (R > 0) {
      // r = x - fp32(L V^T): the product is rounded to fp32 on its own, then subtracted
      // (low_rank_extraction_fuse_compression_quantization.py:72), which also keeps the
      // MFMA independent of x so it issues while x is still in flight.
      const float zero[E] = {};
      float pl[E];
      residual_unit<G, R>(vop[p], lop, zero, pl);
#pragma unroll
      for (int e = 0; e < E; ++e) r[e] = __fsub_rn(r[e], pl[e]);
    }
    if (colmask != nullptr) {
      const int c0 = unit_base(p, u, N, NP, G) + E * g;  // E consecutive columns in one mask word
      const uint32_t mbits = colmask[c0 >> 5] >> (c0 & 31);
#pragma unroll
      for (int e = 0; e < E; ++e)
        if ((mbits >> e) & 1u) r[e] = 0.f;
    }
    float mn = r[0], mx = r[0];
#pragma unroll
    for (int e = 1; e < E; ++e) {
      mn = fminf(mn, r[e]);
      mx = fmaxf(mx, r[e]);
    }
    mn = wave_min4(mn);
    mx = wave_max4(mx);
    const GroupParams gp = group_params<BITS>(mn, mx);
    qp[p] = gp.sh | (gp.zh << 16);
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const uint32_t b = quant_code_bits<BITS>(r[e], gp);  // code in the low BITS bits
      if constexpr (NP == 1) byte[e] = b;
      else if (p == 0) byte[e] = b & 0xfu;
      else byte[e] = (b << 4) | byte[e];
    }
  }
  uint32_t word[E / 4];
#pragma unroll
  for (int i = 0; i < E / 4; ++i) word[i] = gather_bytes(byte[4 * i], byte[4 * i + 1], byte[4 * i + 2], byte[4 * i + 3]);
  // Unconditional stores (see the header comment): all four lanes of a row hold the same
  // (scale, zero) pairs and write them to the same address.
#pragma unroll
  for (int i = 0; i < E / 16; ++i)
    st16(crow + u * G + E * g + 16 * i, u32x4{word[4 * i], word[4 * i + 1], word[4 * i + 2], word[4 * i + 3]});
  if constexpr (NP == 2) st8(qrow + u * 4, u32x2{qp[0], qp[1]});
  else st4(qrow + u * 2, qp[0]);
}

}  // namespace lrq
