// Residual + per-group quantisation of one "unit" of columns, shared by the fused
// single-pass encode and the streaming (second-pass / rank-0) encode.
//
// A unit is, for every packing plane p (NP = 8/BITS planes; plane p holds columns
// [p*N/NP, (p+1)*N/NP)), the CPG = G/32 consecutive chunks starting at chunk `cu` of that
// plane.  Lane (j, g) holds 8 columns of each chunk, so it holds 8*CPG elements of each
// of the NP groups the unit covers; the other three lanes of row j hold the rest, and a
// two-step xor-shuffle finishes the group min/max.
#pragma once

#include "lrq_common.h"

namespace lrq {

template <int BITS, int G, int R>
__device__ __forceinline__ void quant_unit(const u32x4 (&x)[8 / BITS][G / 32], int cu, int PC,
                                           const uint16_t* __restrict__ V, const u32x2* lop,
                                           const uint32_t* colmask, int j, int g, bool rv,
                                           uint8_t* __restrict__ crow, uint16_t* __restrict__ srow,
                                           uint16_t* __restrict__ zrow) {
  constexpr int NP = 8 / BITS, CPG = G / 32;
  uint32_t word[CPG][2];
#pragma unroll
  for (int k = 0; k < CPG; ++k) word[k][0] = word[k][1] = 0u;

#pragma unroll
  for (int p = 0; p < NP; ++p) {
    float r[CPG][8];
    float mn = __builtin_huge_valf(), mx = -__builtin_huge_valf();
#pragma unroll
    for (int k = 0; k < CPG; ++k) {
      const int c0 = (p * PC + cu + k) * 32;
      unpack8(x[p][k], r[k]);
      if constexpr (R > 0) {
        float pl[8];
        lowrank_chunk<R>(V, c0, j, g, lop, pl);
#pragma unroll
        for (int e = 0; e < 8; ++e) r[k][e] = __fsub_rn(r[k][e], pl[e]);
      }
      if (colmask != nullptr) {
        const uint32_t mbits = colmask[c0 >> 5] >> (8 * g);
#pragma unroll
        for (int e = 0; e < 8; ++e)
          if ((mbits >> e) & 1u) r[k][e] = 0.f;
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        mn = fminf(mn, r[k][e]);
        mx = fmaxf(mx, r[k][e]);
      }
    }
    mn = wave_min4(mn);
    mx = wave_max4(mx);
    const GroupParams gp = group_params<BITS>(mn, mx);
    if (rv && g == 0) {
      const int gi = ((p * PC + cu) * 32) / G;
      srow[gi] = gp.sh;
      zrow[gi] = gp.zh;
    }
#pragma unroll
    for (int k = 0; k < CPG; ++k) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const uint32_t c = quant_code<BITS>(r[k][e], gp);
        word[k][e >> 2] |= c << (8 * (e & 3) + BITS * p);
      }
    }
  }
  if (rv) {
#pragma unroll
    for (int k = 0; k < CPG; ++k) {
      u32x2 w2 = {word[k][0], word[k][1]};
      st8(crow + (cu + k) * 32 + 8 * g, w2);
    }
  }
}

}  // namespace lrq
