// Legacy (reference-format) kernels: the arithmetic of the reference's torch forms.
//
//   encode  torch_low_rank_addition_fuse_compression_quantization
//           (low_rank_extraction_fuse_compression_quantization.py:153-171)
//             xr = bf16(x - bf16(l @ r));  o = xr if |xr| > bf16(tau) else 0;
//             c  = clamp(rint(bf16((xr - o) / s)), -2^(b-1), 2^(b-1)-1) + 2^(b-1)
//             q  = row-planar packing: byte j of a row holds column j + p*N/NP in bits
//                  p*b .. p*b+b-1 of plane p (NP = 8/b planes)
//   decode  torch_low_rank_addition_fuse_decompression_dequantization
//           (low_rank_extraction_fuse_decompression_dequantization.py:155-165)
//             x_hat = bf16(bf16(bf16((c - 2^(b-1)) * s) + o) + bf16(l @ r))
//   fused   decode without outliers, then store / SiLU backward / product with y
//           (extraction_fuse_silu_backward.py:192-216, extraction_fuse_hadamard.py:185-209)
//   add     torch_low_rank_addition (low_rank_extraction_speed.py:106-107): bf16(x + bf16(l @ r))
//   hist    histogram of the 15-bit magnitudes |bf16(x - bf16(l @ r))| (the encode's residual), for
//           the outlier threshold torch.kthvalue(|x[0] - l @ r|, k) of
//           low_rank_system_profile_forward.py:45: a 256-bin pass over the top 8 bits, then a
//           128-bin pass over the low 7 bits of the keys in the selected bin.
//
// l is [M, K] and rt = r^T is [N, K] (K = 16 or 32, zero-padded by the caller as the reference
// pads K < 16); s is [1 or B, N].  bf16(l @ r) is the fp32 rounding of the exact sum, then bf16
// (what an fp32-accumulating GEMM returns up to the order of its additions).
//
// Two implementations with identical results:
//   * k_legacy_mfma — when every plane is a whole number of 64-column units and the operands
//     are 16-byte aligned.  The unit layout of lrq_common.h (lane (j, g) owns 16 consecutive
//     columns of its row in every plane) with l @ r rebuilt on MFMA exactly like the
//     group-mode reconstruction (V = rt).
//   * k_legacy_scalar — any shape: one thread per packed byte, l @ r summed in fp64 (the
//     products of bf16 values are exact and so is their fp64 sum for K <= 32).
#include "lrq_common.h"
#include "lrq_coo.h"
#include "lrq_host.h"
#include "lrq_math.h"

namespace lrq {

enum LegacyMode : int { kEncode = 0, kDecode = 1, kFusedStore = 2, kFusedSilu = 3, kFusedMul = 4, kAdd = 5, kHist = 6 };

struct LegacyArgs {
  const uint16_t* l;    // [M, K]
  const uint16_t* rt;   // [N, K]
  const uint16_t* x;    // encode / add input [B, M, N] with strides (ldx_b, ldx_m, 1)
  int64_t ldx_b, ldx_m;
  const uint16_t* s;    // [s_rows, N]
  int64_t s_rows;
  const uint8_t* qin;   // decode / fused codes [B, M, N/NP]
  const uint16_t* oin;  // decode outliers, dense [B, M, N], or null
  const int64_t* optr;  // decode outliers as COO: first entry of each 64-column piece of a row,
  const int64_t* ocol;  //   [B * M * npc + 1]; the entries' column indices and bf16 values, in
  const uint16_t* oval; //   row-major order (lrq_coo_compact's output)
  int64_t npc;          // 64-column pieces per row, ceil(N / 64)
  int64_t* pcnt;        // staged encode: each 64-column piece's record (lrq_coo.h), [B * M * npc]
  int64_t ncap;         // entries the COO arrays hold: reads are clamped to [0, ncap)
  uint32_t* hist;       // hist: 256 global bins
  const int64_t* sel;   // hist: sel[0] = the selected top-8-bit bin, or -1 in the first pass
  const uint16_t* y;    // fused SiLU dy / product operand [B, M, N]
  uint16_t* out;        // decode / fused / add output [B, M, N]
  uint16_t* oout;       // encode outliers, dense [B, M, N]
  uint8_t* qout;        // encode codes [B, M, N/NP]
  int64_t M, N;
  float tau;            // outlier threshold, already rounded to bf16
  int rb;               // MFMA path: 64-row blocks per workgroup
};

// Encode of one element given its bf16 input x, bf16(l @ r) lr and scale sc: returns the code
// (0 .. 2^b - 1) and writes the outlier value (0 unless an outlier).
// big: |xr| > tau, i.e. o = xr; with tau >= 0 that is exactly an outlier entry the compaction
// keeps (o's bf16 bits not +-0).
template <int BITS>
__device__ __forceinline__ uint32_t legacy_code(float x, float lr, float sc, float tau, float& o, bool& big) {
  constexpr float half = (float)(1 << (BITS - 1));
  const float xr = bf16r(x - lr);
  big = fabsf(xr) > tau;
  o = big ? xr : 0.f;
  const float d = bf16r((xr - o) / sc);  // IEEE division, then the bf16 rounding of the torch op
  const float c = __builtin_amdgcn_fmed3f(rintf(d), -half, half - 1.f);
  return (uint32_t)(int)(c + half);
}

// The MFMA encode's forms of legacy_code, with the same codes:
// - the quotient: for scales with 2^-100 <= |sc| <= 2^100 (rc_scale_ok) the one-multiply
//   estimate a * rc, rc = 1/sc rounded once, instead of the IEEE division: its code equals the
//   IEEE quotient's at every bit width for every finite bf16 numerator a (a and sc are bf16
//   values, so a / sc never comes near a code boundary within the estimate's error); other
//   scales take the IEEE division;
// - bf16_roundtrip2 rounds two values to bf16 with one conversion;
// - the code of a bf16 quotient d is legacy_code_biased(d) - kCodeBias + half, where
//   legacy_code_biased(d) = bits(d + 1.5 * 2^23) clamped to [kCodeBias - half, kCodeBias + half - 1]:
//   for |d| < 2^22 the sum lies in [2^23, 2^24), where the fp32 ulp is 1, so the add rounds d to the
//   nearest integer, ties to even (1.5 * 2^23 is even), as rint does, and the bits are kCodeBias +
//   rint(d); for d >= 2^22 the sum is at least 2^24 and clamps to the top code; for d <= -2^22 it is
//   at most 2^23, +0 or negative (a negative int32) and clamps to the bottom code, as the clamp of
//   rint(d) does (infinities included).  A byte starting from legacy_code_base (the sum of
//   (half - kCodeBias) << BITS p over its planes, mod 2^32) and adding legacy_code_biased << BITS p
//   per plane holds the planes' codes in its low 8 bits;
// - at 1 bit the code is 1 exactly when bf16(q) >= -0.5, i.e. when q >= -(0.5 + 2^-9) (below
//   -0.5 the bf16 spacing is 2^-8, and the tie at -0.5 - 2^-9 rounds to the even -0.5): one
//   compare of the quotient, no rounding.
// The host check tests/legacy_code_check.c compares the code forms with the reference's over
// every fp32 quotient but NaN, and the estimate's codes with the IEEE quotient's at 1, 2, 4 and
// 8 bits over every finite bf16 numerator and every scale the estimate serves.
constexpr uint32_t kCodeBias = 0x4B400000u;  // bits of 1.5 * 2^23
template <int BITS>
__device__ __forceinline__ uint32_t legacy_code_biased(float d) {
  constexpr int half = 1 << (BITS - 1);
  const int v = (int)__float_as_uint(d + 0x1.8p23f);
  return (uint32_t)min(max(v, (int)kCodeBias - half), (int)kCodeBias + half - 1);
}
constexpr float kOneBitLow = -(0.5f + 0x1p-9f);
template <int BITS>
constexpr uint32_t legacy_code_base() {
  if (BITS == 1) return 0u;  // the 1-bit codes are or-ed in
  uint32_t k = 0;
  for (int p = 0; p < 8 / BITS; ++p) k += ((1u << (BITS - 1)) - kCodeBias) << (BITS * p);
  return k;
}

// legacy_code of two elements for the MFMA encode, in the forms above (RC: the estimate of the
// quotient, else the IEEE division), with one bf16 conversion per rounding step of the pair: at
// 1 bit the code itself (an outlier leaves a = 0, whose code is 1; otherwise a = xr), at 2, 4
// and 8 bits biased (legacy_code_biased).
template <int BITS, bool RC>
__device__ __forceinline__ void legacy_code_mfma2(const float* x, const float* lr, const float* sc, const float* rc,
                                                  float tau, float* o, bool* big, uint32_t* code) {
  float xr[2] = {x[0] - lr[0], x[1] - lr[1]}, q[2];
  bf16_roundtrip2(xr[0], xr[1]);
  if constexpr (BITS == 1) {
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      big[k] = fabsf(xr[k]) > tau;
      o[k] = big[k] ? xr[k] : 0.f;
      const float qk = RC ? xr[k] * rc[k] : xr[k] / sc[k];  // (IEEE division when !RC)
      code[k] = (big[k] || qk >= kOneBitLow) ? 1u : 0u;
    }
    return;
  }
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    big[k] = fabsf(xr[k]) > tau;
    o[k] = big[k] ? xr[k] : 0.f;
    const float a = xr[k] - o[k];
    q[k] = RC ? a * rc[k] : a / sc[k];  // (IEEE division when !RC)
  }
  bf16_roundtrip2(q[0], q[1]);
  code[0] = legacy_code_biased<BITS>(q[0]);
  code[1] = legacy_code_biased<BITS>(q[1]);
}
template <int BITS>
__device__ __forceinline__ void legacy_accumulate(uint32_t& byte, uint32_t code, int p) {
  if constexpr (BITS == 1) byte |= code << p;
  else byte += code << (BITS * p);
}

// The bf16 bits of element i (0 .. 15) of the 16 packed in w0 (elements 0 .. 7) and w1: a select
// tree, no indexed register access.
__device__ __forceinline__ uint32_t bf16_at(const u32x4& w0, const u32x4& w1, uint32_t i) {
  const u32x4 w = (i & 8u) ? w1 : w0;
  const uint32_t lo = (i & 2u) ? w[1] : w[0], hi = (i & 2u) ? w[3] : w[2];
  const uint32_t d = (i & 4u) ? hi : lo;
  return (d >> (16u * (i & 1u))) & 0xffffu;
}

// Scales whose reciprocal estimate gives legacy_code's codes (NaN fails the test).
__device__ __forceinline__ bool rc_scale_ok(float sc) {
  const float m = fabsf(sc);
  return m >= 0x1p-100f && m <= 0x1p100f;
}

// Decode of one element: bf16(bf16(bf16((code - 2^(b-1)) * s) + o) + lr); with !HAS_O the add
// of o (exact zero) is skipped.  The outliers come as a dense tensor (OSRC 1) or as COO pieces
// (OSRC 2); both feed the same per-element add, so the two give the same bits.
template <int BITS, bool HAS_O>
__device__ __forceinline__ float legacy_value(uint32_t code, float sc, float o, float lr) {
  float a = bf16r((float)((int)code - (1 << (BITS - 1))) * sc);
  if constexpr (HAS_O) a = bf16r(a + o);
  return bf16r(a + lr);
}

// Histogram bin of a residual xr (bf16 value) for the pass that sel selects, or -1 if the key
// is not counted in this pass.
__device__ __forceinline__ int hist_bin(float xr, int64_t sel) {
  const uint32_t key = (__float_as_uint(xr) >> 16) & 0x7fffu;
  if (sel < 0) return (int)(key >> 7);
  return (int64_t)(key >> 7) == sel ? (int)(key & 127u) : -1;
}

template <int MODE>
__device__ __forceinline__ float legacy_consume(float xh, float yv) {
  if constexpr (MODE == kFusedSilu) return silu_bwd_f32(xh, yv);
  else if constexpr (MODE == kFusedMul) return xh * yv;
  else return xh;
}

// The outlier values of columns c0 .. c0 + E - 1 of row `bm` (b * M + m) from the COO pieces
// (sparse outliers, OSRC 2): the entries of the piece holding c0 (the E columns never straddle a
// piece boundary), one at a time.
template <int E>
__device__ __forceinline__ void coo_piece_values(const LegacyArgs& a, int64_t bm, int64_t c0, float* oo) {
#pragma unroll
  for (int e = 0; e < E; ++e) oo[e] = 0.f;
  const int64_t pc = bm * a.npc + c0 / 64;
  const int64_t e1 = min(a.optr[pc + 1], a.ncap);
  for (int64_t k = max(a.optr[pc], (int64_t)0); k < e1; ++k) {
    const int64_t d = a.ocol[k] - c0;
    const float v = __uint_as_float((uint32_t)a.oval[k] << 16);
#pragma unroll
    for (int e = 0; e < E; ++e) oo[e] = d == e ? v : oo[e];
  }
}

// Denser outliers (OSRC 3): the COO pieces of a wave's 16 rows x one unit (NP pieces of 64
// columns per row) go into the wave's
// LDS tile ot[row][plane][64] (bf16 bits).  The four lanes of a row share its pieces: the piece
// bounds come from coo_bounds (requested a block ahead), then in each pass lane (j, g) requests entries
// g, g + 4, .. (KL per piece) of each of its row's pieces, all of them before any is used
// (clamped indices; no load sits under a branch), and writes those that fall in the piece into
// the tile after the lane has zeroed its own 16 columns of every plane.  Another pass runs only
// while some piece of the wave has more entries.  Entries of a coalesced COO are unique per
// position (so no two lanes write the same one), and entries outside the piece are ignored.
// The piece bounds of row bm's NP pieces of unit u (requested together; coo_tile uses them).
template <int NP>
__device__ __forceinline__ void coo_bounds(const LegacyArgs& a, int64_t bm, int u, int N, int64_t (&s0)[NP],
                                           int64_t (&s1)[NP]) {
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    const int64_t pc = bm * a.npc + (int64_t)(p * (N / NP) + u * 64) / 64;
    s0[p] = a.optr[pc];
    s1[p] = a.optr[pc + 1];
  }
}

// Entries each lane requests per piece and pass (4 lanes per row: 4 * KL entries of a piece per pass).
static constexpr int kCooEntriesPerLane = 2;
// bf16 of padding after each row of the COO tile: rows 16 bytes apart in the LDS banks, so the
// 16-byte accesses of 8 consecutive lanes (8 rows) fall in distinct banks.
static constexpr int kCooRowPad = 8;
template <int NP>
constexpr int coo_row_stride() { return NP * 64 + kCooRowPad; }
template <int NP, int KL>
__device__ __forceinline__ void coo_tile(const LegacyArgs& a, int64_t (&s0)[NP], int64_t (&s1)[NP], int u, int N,
                                         int j, int g, uint16_t* __restrict__ ot) {
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    uint16_t* r = ot + j * coo_row_stride<NP>() + p * 64 + 16 * g;
    st16(r, u32x4{0u, 0u, 0u, 0u});
    st16(r + 8, u32x4{0u, 0u, 0u, 0u});
    s0[p] = max(s0[p], (int64_t)0);
    s1[p] = min(s1[p], a.ncap);
  }
  if (a.ncap <= 0) return;  // uniform: no entries at all
  const uint32_t* col32 = reinterpret_cast<const uint32_t*>(a.ocol);  // low dword of each int64 column
  for (int pass = 0;; ++pass) {
    uint32_t cv[NP][KL];
    uint16_t vv[NP][KL];
#pragma unroll
    for (int p = 0; p < NP; ++p)
#pragma unroll
      for (int i = 0; i < KL; ++i) {
        const int64_t k = min(s0[p] + (int64_t)(4 * KL * pass + g + 4 * i), a.ncap - 1);
        cv[p][i] = col32[2 * k];
        vv[p][i] = a.oval[k];
      }
    bool more = false;
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      const int64_t base = p * (N / NP) + u * 64;
#pragma unroll
      for (int i = 0; i < KL; ++i) {
        const int64_t k = s0[p] + (int64_t)(4 * KL * pass + g + 4 * i);
        const int64_t d = (int64_t)cv[p][i] - base;
        if (k < s1[p] && d >= 0 && d < 64) ot[j * coo_row_stride<NP>() + p * 64 + (int)d] = vv[p][i];
      }
      more |= s1[p] - s0[p] > (int64_t)4 * KL * (pass + 1);
    }
    if (!__builtin_amdgcn_ballot_w64(more)) break;  // uniform
  }
}

// ------------------------------------------------------------------ MFMA path
// Grid: ceil(M / (64 * rb)) * (N / (64 * NP)) * B workgroups (one dimension); 4 waves; the
// workgroup's tile t = (b, bx, u), units fastest, is xcd_tile of its index: the workgroups of one
// XCD that run together cover neighbouring units of the same rows, which share L2 lines of the COO
// entries (a piece's entries do not start on a line boundary), of the code rows and of the output
// rows.  Wave w walks row blocks (bx * rb + i) * 64 + w * 16, i < rb, of unit u.  OSRC, decode: outliers
// absent (0), dense (1) or COO pieces (2: looked up per lane, for sparse outliers; 3: gathered
// per wave into an LDS tile, for denser ones); encode: 1 writes each 64-column piece's staged
// record (a.pcnt; lrq_coo.h) and the dense outliers only of the pieces it cannot hold.
template <int MODE, int BITS, int K, int OSRC>
__global__ __launch_bounds__(256) void k_legacy_mfma(LegacyArgs a) {
  constexpr int NP = (MODE == kAdd || MODE == kHist) ? 1 : 8 / BITS, G = 64, E = 16, RT = K / 16;
  __shared__ uint32_t lh[MODE == kHist ? 256 : 1];
  // decode from denser COO outliers: each wave's outlier tile (16 rows x NP planes x 64 columns, bf16)
  __shared__ __attribute__((aligned(16))) uint16_t otile[(MODE == kDecode && OSRC == 3) ? 4 * 16 * coo_row_stride<NP>() : 8];
  int64_t sel = -1;
  if constexpr (MODE == kHist) {
    lh[threadIdx.x] = 0u;
    sel = a.sel[0];
    __syncthreads();
  }
  constexpr uint32_t kMask = BITS == 8 ? 0xffu : (1u << BITS) - 1u;
  const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
  const int j = lane & 15, g = lane >> 4;
  const int M = (int)a.M, N = (int)a.N;
  // tile t = (batch, 64-row chunk, unit), units fastest
  const int nu = N / NP / G, gx = (M + 64 * a.rb - 1) / (64 * a.rb);
  const int t = __builtin_amdgcn_readfirstlane(xcd_tile(blockIdx.x, gridDim.x));
  const int u = __builtin_amdgcn_readfirstlane(t % nu);
  const int bx = __builtin_amdgcn_readfirstlane((t / nu) % gx);
  const int b = __builtin_amdgcn_readfirstlane(t / (nu * gx));
  const int64_t NB = N / NP;  // bytes per code row
  const uint16_t* srow = a.s + (a.s_rows == 1 ? 0 : (int64_t)b * N);

  u32x2 vop[NP][G / 16][RT];
#pragma unroll
  for (int p = 0; p < NP; ++p) load_vops<G, K>(a.rt, unit_base(p, u, N, NP, G), j, g, vop[p]);
  const float zero[E] = {};

  // the unit's scales in LDS for every row block of the workgroup (the same columns throughout),
  // and for the encode their reciprocals (one IEEE division per column); rc_ok: every scale is
  // the reciprocal estimate serves exactly
  constexpr bool kScales = MODE != kAdd && MODE != kHist;
  __shared__ __attribute__((aligned(16))) float stab[MODE == kEncode ? 2 * NP * G : (kScales ? NP * G : 4)];
  bool rc_ok = false;
  if constexpr (kScales) {
    int ok = 1;
    for (int i = threadIdx.x; i < NP * G; i += 256) {
      const int p = i / G, c = i % G;
      const float sv = bf_lo(srow[unit_base(p, u, N, NP, G) + c]);
      stab[i] = sv;
      if constexpr (MODE == kEncode) {
        stab[NP * G + i] = 1.0f / sv;
        ok &= rc_scale_ok(sv) ? 1 : 0;
      }
    }
    if constexpr (MODE == kEncode) {
      // every thread's ok, as __syncthreads_and (whose device-library reduction is not inlined
      // here): one ballot per wave, the 4 waves' results through LDS
      __shared__ uint32_t wave_ok[4];
      const bool all = __builtin_amdgcn_ballot_w64(ok == 0) == 0;
      if (lane == 0) wave_ok[w] = all ? 1u : 0u;
      __syncthreads();
      rc_ok = (wave_ok[0] & wave_ok[1] & wave_ok[2] & wave_ok[3]) != 0;
    } else {
      __syncthreads();
    }
  }

  // decode from the COO tile: the next row block's L operand, codes and COO piece bounds are
  // requested before the current block is computed (nl / nq / ns0 / ns1 carry them over; the
  // other modes measured slower with the carried registers)
  constexpr bool kCodes = MODE == kDecode || MODE == kFusedStore || MODE == kFusedSilu || MODE == kFusedMul;
  constexpr bool kPre = MODE == kDecode && OSRC == 3;
  constexpr int NPB = (MODE == kDecode && OSRC == 3) ? NP : 1;  // COO piece bounds per lane
  u32x2 nl[RT];
  u32x4 nq = u32x4{0u, 0u, 0u, 0u};
  int64_t ns0[NPB], ns1[NPB];
  auto fetch_next = [&](int i) __attribute__((always_inline)) {  // block i of the workgroup (rows clamped to the last)
    const int64_t rn = min((bx * a.rb + i) * 64 + w * 16 + j, M - 1);
#pragma unroll
    for (int t = 0; t < RT; ++t) nl[t] = ld8(a.l + rn * K + 16 * t + 4 * g);
    nq = ld16(a.qin + ((int64_t)b * M + rn) * NB + u * G + E * g);
    if constexpr (MODE == kDecode && OSRC == 3) coo_bounds<NP>(a, (int64_t)b * M + rn, u, N, ns0, ns1);
  };
  if constexpr (kPre) fetch_next(0);
  // encode at 2 bits and more: the next row block's x (and L operand) is requested before the
  // current block is computed (nx carries it over; at 1 bit its 64 registers would halve the
  // waves per SIMD)
  constexpr bool kPreX = MODE == kEncode && NP <= 4;
  u32x4 nx[kPreX ? NP : 1][2];
  auto fetch_x = [&](int i) __attribute__((always_inline)) {
    const int64_t rn = min((bx * a.rb + i) * 64 + w * 16 + j, M - 1);
#pragma unroll
    for (int t = 0; t < RT; ++t) nl[t] = ld8(a.l + rn * K + 16 * t + 4 * g);
#pragma unroll
    for (int p = 0; p < (kPreX ? NP : 1); ++p) {
      const uint16_t* xp = a.x + (int64_t)b * a.ldx_b + rn * a.ldx_m + unit_base(p, u, N, NP, G) + E * g;
      nx[p][0] = ld16(xp);
      nx[p][1] = ld16(xp + 8);
    }
  };
  if constexpr (kPreX) fetch_x(0);

  for (int i = 0; i < a.rb; ++i) {
    const int row0 = (bx * a.rb + i) * 64 + w * 16;  // wave-uniform: a scalar exit
    if (row0 >= M) break;  // whole 16-row block past the end
    const int row = row0 + j;
    const int64_t rr = min(row, M - 1);
    const int64_t erow = ((int64_t)b * M + rr) * N;  // element offset of the row in [B, M, N] outputs
    u32x2 lop[RT];
    u32x4 qb = u32x4{0u, 0u, 0u, 0u};
    int64_t s0[NPB], s1[NPB];
    if constexpr (kPre) {
#pragma unroll
      for (int t = 0; t < RT; ++t) lop[t] = nl[t];
      qb = nq;
#pragma unroll
      for (int q = 0; q < NPB; ++q) {
        s0[q] = ns0[q];
        s1[q] = ns1[q];
      }
      fetch_next(min(i + 1, a.rb - 1));  // (the last block fetches itself again: unused)
    } else if constexpr (kPreX) {
#pragma unroll
      for (int t = 0; t < RT; ++t) lop[t] = nl[t];
    } else {
#pragma unroll
      for (int t = 0; t < RT; ++t) lop[t] = ld8(a.l + rr * K + 16 * t + 4 * g);
      if constexpr (kCodes) qb = ld16(a.qin + ((int64_t)b * M + rr) * NB + u * G + E * g);
    }
    u32x4 cx[kPreX ? NP : 1][2];
    if constexpr (kPreX) {
#pragma unroll
      for (int p = 0; p < NP; ++p) {
        cx[p][0] = nx[p][0];
        cx[p][1] = nx[p][1];
      }
      fetch_x(min(i + 1, a.rb - 1));  // (the last block fetches itself again: unused)
    }
    uint32_t byte[E];
#pragma unroll
    for (int e = 0; e < E; ++e) byte[e] = MODE == kEncode ? legacy_code_base<BITS>() : 0u;
    uint16_t* ot = otile + (size_t)w * 16 * coo_row_stride<NP>();
    if constexpr (MODE == kDecode && OSRC == 3) coo_tile<NP, kCooEntriesPerLane>(a, s0, s1, u, N, j, g, ot);

#pragma unroll
    for (int p = 0; p < NP; ++p) {
      const int c0 = unit_base(p, u, N, NP, G) + E * g;
      float lr[E];
      residual_unit<G, K>(vop[p], lop, zero, lr);
#pragma unroll
      for (int e = 0; e < E; e += 2) bf16_roundtrip2(lr[e], lr[e + 1]);
      float sc[E], rc[E];
      if constexpr (MODE == kEncode) {
        const float* sp = stab + p * G + E * g;
#pragma unroll
        for (int k = 0; k < E; k += 4) {
          const f32x4 v = *reinterpret_cast<const f32x4*>(sp + k);
          const f32x4 w = *reinterpret_cast<const f32x4*>(sp + NP * G + k);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            sc[k + e] = v[e];
            rc[k + e] = w[e];
          }
        }
      } else if constexpr (kScales) {
        const float* sp = stab + p * G + E * g;
#pragma unroll
        for (int k = 0; k < E; k += 4) {
          const f32x4 v = *reinterpret_cast<const f32x4*>(sp + k);
#pragma unroll
          for (int e = 0; e < 4; ++e) sc[k + e] = v[e];
        }
      }
      if constexpr (MODE == kHist) {
        float xv[E];
        const uint16_t* xp = a.x + rr * a.ldx_m + c0;
        unpack8(ld16(xp), xv);
        unpack8(ld16(xp + 8), xv + 8);
        if (row < M) {
#pragma unroll
          for (int e = 0; e < E; ++e) {
            const int bin = hist_bin(bf16r(xv[e] - lr[e]), sel);
            if (bin >= 0) atomicAdd(&lh[bin], 1u);
          }
        }
      } else if constexpr (MODE == kEncode || MODE == kAdd) {
        float xv[E];
        if constexpr (kPreX) {
          unpack8(cx[p][0], xv);
          unpack8(cx[p][1], xv + 8);
        } else {
          const uint16_t* xp = a.x + (int64_t)b * a.ldx_b + rr * a.ldx_m + c0;
          unpack8(ld16(xp), xv);
          unpack8(ld16(xp + 8), xv + 8);
        }
        if constexpr (MODE == kEncode) {
          // legacy_code of each element in the forms above, two at a time (legacy_code_mfma2)
          float ov[E];
          uint32_t hm = 0;  // bit e: element e is an outlier entry
          if (rc_ok) {  // workgroup-uniform
#pragma unroll
            for (int e = 0; e < E; e += 2) {
              bool hit[2];
              uint32_t cd[2];
              legacy_code_mfma2<BITS, true>(xv + e, lr + e, sc + e, rc + e, a.tau, ov + e, hit, cd);
              legacy_accumulate<BITS>(byte[e], cd[0], p);
              legacy_accumulate<BITS>(byte[e + 1], cd[1], p);
              hm |= (hit[0] ? 1u << e : 0u) | (hit[1] ? 2u << e : 0u);
            }
          } else {
#pragma unroll
            for (int e = 0; e < E; e += 2) {
              bool hit[2];
              uint32_t cd[2];
              legacy_code_mfma2<BITS, false>(xv + e, lr + e, sc + e, rc + e, a.tau, ov + e, hit, cd);
              legacy_accumulate<BITS>(byte[e], cd[0], p);
              legacy_accumulate<BITS>(byte[e + 1], cd[1], p);
              hm |= (hit[0] ? 1u << e : 0u) | (hit[1] ? 2u << e : 0u);
            }
          }
          const u32x4 ow0 = pack8(ov), ow1 = pack8(ov + 8);
          if constexpr (OSRC == 1) {
            // the piece's staged record (lrq_coo.h): its count and first kCooSlots entries, over
            // the row's four lanes (lane g holds the piece's columns 16g .. 16g+15); its dense
            // values only when the record cannot hold them
            const uint32_t n = __builtin_popcount(hm);
            uint32_t pre, total;
            row_prefix4(n, g, pre, total);
            const uint32_t i0 = __builtin_ctz(hm | 0x10000u) & 15u, h1 = hm & (hm - 1u);
            const uint32_t i1 = __builtin_ctz(h1 | 0x10000u) & 15u;
            const uint32_t e0 = ((uint32_t)(16 * g) + i0) | (bf16_at(ow0, ow1, i0) << 16);
            const uint32_t e1 = ((uint32_t)(16 * g) + i1) | (bf16_at(ow0, ow1, i1) << 16);
            static_assert(kCooSlots == 2, "two entries per record");
            uint32_t d0 = pre == 0u && n >= 1u ? e0 : 0u;
            uint32_t d1 = pre == 0u && n >= 2u ? e1 : pre == 1u && n >= 1u ? e0 : 0u;
            d0 = row_or4(d0);
            d1 = row_or4(d1);
            // lane g = 0 of each row stores the record through a range-checked store (the other
            // lanes' offsets fall outside the range: no branch)
            int64_t* prow = a.pcnt + ((int64_t)b * M + row0) * a.npc;  // the block's first row
            st8_pred(prow, (uint32_t)(16 * a.npc * 8),
                     (uint32_t)(((rr - row0) * a.npc + unit_base(p, u, N, NP, G) / 64) * 8),
                     u32x2{d0 | total << 8, d1}, g == 0 && row < M);
            uint16_t* orow = a.oout + ((int64_t)b * M + row0) * N;
            const uint32_t olen = (uint32_t)(16 * N * 2), ooff = (uint32_t)(((rr - row0) * N + c0) * 2);
            const bool dense = total > (uint32_t)kCooSlots && row < M;
            st16_pred(orow, olen, ooff, ow0, dense);
            st16_pred(orow, olen, ooff + 16, ow1, dense);
          } else {
            st16(a.oout + erow + c0, ow0);
            st16(a.oout + erow + c0 + 8, ow1);
          }
        } else {
          float ov[E];
#pragma unroll
          for (int e = 0; e < E; ++e) ov[e] = xv[e] + lr[e];  // fp32 add, then bf16 (pack8), as torch
          st16(a.out + erow + c0, pack8(ov));
          st16(a.out + erow + c0 + 8, pack8(ov + 8));
        }
      } else {
        float ov[E], oo[E], yv[E];
        if constexpr (MODE == kDecode && OSRC == 1) {
          unpack8(ld16(a.oin + erow + c0), oo);
          unpack8(ld16(a.oin + erow + c0 + 8), oo + 8);
        }
        if constexpr (MODE == kDecode && OSRC == 2) coo_piece_values<E>(a, (int64_t)b * M + rr, c0, oo);
        if constexpr (MODE == kDecode && OSRC == 3) {
          const uint16_t* r = ot + j * coo_row_stride<NP>() + p * 64 + 16 * g;
          unpack8(*reinterpret_cast<const u32x4*>(r), oo);
          unpack8(*reinterpret_cast<const u32x4*>(r + 8), oo + 8);
        }
        if constexpr (MODE == kFusedSilu || MODE == kFusedMul) {
          unpack8(ld16(a.y + erow + c0), yv);
          unpack8(ld16(a.y + erow + c0 + 8), yv + 8);
        }
#pragma unroll
        for (int e = 0; e < E; ++e) {
          const uint32_t code = (qb[e >> 2] >> (8 * (e & 3) + BITS * p)) & kMask;
          const float xh = legacy_value<BITS, MODE == kDecode && OSRC != 0>(code, sc[e], oo[e], lr[e]);
          ov[e] = legacy_consume<MODE>(xh, yv[e]);
        }
        st16(a.out + erow + c0, pack8(ov));
        st16(a.out + erow + c0 + 8, pack8(ov + 8));
      }
    }
    if constexpr (MODE == kEncode) {
      uint32_t word[E / 4];
#pragma unroll
      for (int k = 0; k < E / 4; ++k) word[k] = gather_bytes(byte[4 * k], byte[4 * k + 1], byte[4 * k + 2], byte[4 * k + 3]);
      st16(a.qout + ((int64_t)b * M + rr) * NB + u * G + E * g, u32x4{word[0], word[1], word[2], word[3]});
    }
  }
  if constexpr (MODE == kHist) {
    __syncthreads();
    if (lh[threadIdx.x] != 0u) atomicAdd(&a.hist[threadIdx.x], lh[threadIdx.x]);
  }
}

// ------------------------------------------------------------------ scalar path
// One thread per packed byte position c of one row; grid.x enumerates (b, m, 256-byte chunk).
template <int MODE, int BITS, int OSRC>
__global__ __launch_bounds__(256) void k_legacy_scalar(LegacyArgs a, int K, int64_t chunks) {
  constexpr int NP = (MODE == kAdd) ? 1 : 8 / BITS;
  constexpr uint32_t kMask = BITS == 8 ? 0xffu : (1u << BITS) - 1u;
  const int64_t M = a.M, N = a.N, NB = N / NP;
  const int64_t blk = blockIdx.x;
  const int64_t bm = blk / chunks;
  const int64_t c = (blk - bm * chunks) * 256 + threadIdx.x;
  if (c >= NB) return;
  const int64_t b = bm / M, m = bm - b * M;
  const uint16_t* srow = a.s + (a.s_rows == 1 ? 0 : b * N);
  const uint16_t* lrow = a.l + m * K;
  const int64_t erow = bm * N;
  uint32_t byte = 0u;
  if constexpr (MODE == kDecode || MODE == kFusedStore || MODE == kFusedSilu || MODE == kFusedMul)
    byte = a.qin[bm * NB + c];
  uint32_t qout = 0u;
  for (int p = 0; p < NP; ++p) {
    const int64_t col = p * NB + c;
    const uint16_t* rrow = a.rt + col * K;
    double acc = 0.0;
    for (int k = 0; k < K; ++k)
      acc = __builtin_fma((double)__uint_as_float((uint32_t)lrow[k] << 16),
                          (double)__uint_as_float((uint32_t)rrow[k] << 16), acc);
    const float lr = bf16r((float)acc);
    if constexpr (MODE == kEncode) {
      const float xv = __uint_as_float((uint32_t)a.x[b * a.ldx_b + m * a.ldx_m + col] << 16);
      const float sc = __uint_as_float((uint32_t)srow[col] << 16);
      float o;
      bool hit;
      qout |= legacy_code<BITS>(xv, lr, sc, a.tau, o, hit) << (BITS * p);
      a.oout[erow + col] = (uint16_t)pack_bf16x2(o, 0.f);
    } else if constexpr (MODE == kAdd) {
      const float xv = __uint_as_float((uint32_t)a.x[b * a.ldx_b + m * a.ldx_m + col] << 16);
      a.out[erow + col] = (uint16_t)pack_bf16x2(xv + lr, 0.f);
    } else {
      const float sc = __uint_as_float((uint32_t)srow[col] << 16);
      const uint32_t code = (byte >> (BITS * p)) & kMask;
      float o = 0.f, yv = 0.f;
      if constexpr (MODE == kDecode && OSRC == 1) o = __uint_as_float((uint32_t)a.oin[erow + col] << 16);
      if constexpr (MODE == kDecode && OSRC >= 2) {  // COO pieces (both lookups give the same values)
        const int64_t pc = bm * a.npc + col / 64, e1 = min(a.optr[pc + 1], a.ncap);
        for (int64_t k = max(a.optr[pc], (int64_t)0); k < e1; ++k)
          if (a.ocol[k] == col) o = __uint_as_float((uint32_t)a.oval[k] << 16);
      }
      if constexpr (MODE == kFusedSilu || MODE == kFusedMul) yv = __uint_as_float((uint32_t)a.y[erow + col] << 16);
      const float xh = legacy_value<BITS, MODE == kDecode && OSRC != 0>(code, sc, o, lr);
      a.out[erow + col] = (uint16_t)pack_bf16x2(legacy_consume<MODE>(xh, yv), 0.f);
    }
  }
  if constexpr (MODE == kEncode) a.qout[bm * NB + c] = (uint8_t)qout;
}

// ------------------------------------------------------------------ row-tile decode
// Decode for large shapes (2, 4 or 8 bits; no outliers, or COO outliers), staged through an LDS
// tile so that the output leaves as whole row segments.  A workgroup of 4 waves owns 4 units
// (wave w: unit u0 + w, i.e. 64 columns in every plane) of one batch over a run of RBW 16-row
// blocks, with the unit's r^T operands in registers and the units' scales in LDS for the whole
// run (in registers they pushed the 2-bit kernel past 256 VGPRs: one wave per SIMD).  The tile is
// [16 rows][NP planes][256 columns] bf16 (rows padded by 16 bytes, so the lanes of a column
// quarter reach different banks), two of them in turn.  Per block b:
//   B1 | x_hat of block b: each lane reads its 16 outlier values per plane from tile b, forms
//   x_hat (the reconstruction MFMA for l @ r, the decode's roundings two columns at a time) and
//   writes it over them; the workers zero the other tile | B2 | tile b leaves as row segments
//   (non-temporal 16-byte stores of whole lines) and the codes and l operand of block b + PD are
//   requested (PD = 2; 4 measured slower); the workers write block b + 1's COO entries, requested
//   a block earlier, into the zeroed tile and request the entries of block b + 2 and the COO
//   bounds of block b + 4.
// COO ranges: the entries of one (row, plane) of the workgroup's units are contiguous (row-major
// COO, 64-column pieces in order): [piece_ptr[pc], piece_ptr[pc + units]).  With outliers the
// workgroup has 4 more waves, COO workers (their loads and waits stay out of the decoding waves'
// in-order memory queues): worker w takes ranges w * RPW .. w * RPW + RPW - 1 (range q: row q % 16,
// plane q / 16), LPR = 64 / RPW lanes each; lane l of range r loads its own bounds and entries
// start + l % LPR + LPR i for the i < ns the wave's longest range needs (64 entries of a range per
// pass); a range of more than 64 entries takes further passes right away.  An entry outside the
// units' columns, or past the entry capacity, is not written.  (Four waves per SIMD, two
// workgroups per CU: 128 VGPRs with a small spill measured faster than 136 VGPRs and one
// workgroup.)  Blocks are taken PD at a time
// (ring slots by position); the positions past the run compute on the last block's inputs and
// store nothing (a zero-length store range).
template <int BITS>
struct LegacyRows {
  static constexpr int NP = 8 / BITS, NW = 4, G = 64, SEG = NW * G, PD = 2;
  static constexpr int RSTR = NP * SEG + 8;  // bf16 per tile row
  static constexpr int TILE = 16 * RSTR;     // bf16 per tile
  static constexpr int NR = 16 * NP, RPW = NR / NW;
  static constexpr size_t LDS = (2 * (size_t)TILE + 64 + NP * SEG) * 2;  // two tiles, a 64-lane dummy row, the scales
  static_assert(BITS == 2 || BITS == 4 || BITS == 8, "2, 4 or 8 bits");
};

template <int BITS, int K, bool COO>
__global__ __launch_bounds__(COO ? 512 : 256) __attribute__((amdgpu_waves_per_eu(4))) void k_legacy_rows(LegacyArgs a, int RBW, int ug) {
  using Lr = LegacyRows<BITS>;
  constexpr int NP = Lr::NP, NW = Lr::NW, G = 64, E = 16, RT = K / 16, SEG = Lr::SEG, RSTR = Lr::RSTR;
  constexpr int TILE = Lr::TILE, RPW = Lr::RPW, PD = Lr::PD, T = COO ? 512 : 256;
  constexpr uint32_t kMask = BITS == 8 ? 0xffu : (1u << BITS) - 1u;
  extern __shared__ __attribute__((aligned(16))) uint16_t lt[];  // [2][TILE] + dummy[64]
  uint16_t* const dummy = lt + 2 * TILE;
  const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int j = lane & 15, g = lane >> 4;
  const int M = (int)a.M, N = (int)a.N;
  const int64_t NB = N / NP;
  const int nu = (int)(NB / G), nrb = (M + 15) / 16, nrun = (nrb + RBW - 1) / RBW;
  // tile (batch, run, unit group), unit groups fastest, in XCD-aware order: the workgroups that
  // run together on an XCD take neighbouring unit groups of the same rows (their COO ranges and
  // code rows share L2 lines)
  const int t = __builtin_amdgcn_readfirstlane(xcd_tile(blockIdx.x, gridDim.x));
  const int ugi = t % ug, run = (t / ug) % nrun, b = t / (ug * nrun);
  const int u0 = ugi * NW, nuw = min(NW, nu - u0), u = min(u0 + w % NW, nu - 1);
  // with COO outliers, waves NW .. 2 NW - 1 are COO workers: they zero the tiles and write the
  // entries into them, so that their loads and waits never hold up the decoding waves' block ring
  // (memory operations retire in issue order, per wave)
  const bool worker = COO && w >= NW;  // (uniform)
  const int rb0 = run * RBW, nblk = min(RBW, nrb - rb0);
  const int64_t bm0 = (int64_t)b * M;  // first row of the batch in [B * M] rows
  const uint16_t* srow = a.s + (a.s_rows == 1 ? 0 : (int64_t)b * N);

  // resident: the unit's r^T operands and its 16 scales per plane (bf16 pairs)
  u32x2 vop[NP][G / 16][RT];
  uint16_t* const stab = lt + 2 * TILE + 64;  // [NP][SEG] scales of the workgroup's units (bf16)
  if (!worker) {
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      const int base = unit_base(p, u, N, NP, G);
      load_vops<G, K>(a.rt, base, j, g, vop[p]);
    }
  }
  for (int i = threadIdx.x; i < NP * SEG; i += T) {
    const int p = i / SEG, c = min(i % SEG, nuw * G - 1);
    stab[i] = srow[p * (int)NB + u0 * G + c];
  }

  // per block: codes (16 bytes per lane) and the l operand, PD blocks ahead
  struct Blk {
    u32x4 cb;
    u32x2 lop[RT];
  };
  auto load_blk = [&](int i, Blk& d) __attribute__((always_inline)) {
    const int64_t rr = min(min(rb0 + i, nrb - 1) * 16 + j, M - 1);
    d.cb = ld16_stream(a.qin + (bm0 + rr) * NB + u * G + E * g);
#pragma unroll
    for (int k = 0; k < RT; ++k) d.lop[k] = ld8(a.l + rr * K + 16 * k + 4 * g);
  };
  // COO (workers): this lane's range (row rq, plane pq) and its place among the range's LPR lanes
  constexpr int LPR = 64 / RPW;
  const int wq = w % NW;
  const int rq = (wq * RPW + lane / LPR) % 16, pq = (wq * RPW + lane / LPR) / 16, lr_ = lane % LPR;
  const int cbase = pq * (int)NB + u0 * G;  // the range's first column
  struct Bnd {
    int64_t s0, s1;
  };
  auto load_bounds = [&](int i) __attribute__((always_inline)) -> Bnd {
    const int64_t rr = min(min(rb0 + i, nrb - 1) * 16 + rq, M - 1);
    const int64_t pc = (bm0 + rr) * a.npc + (int64_t)pq * (NB / G) + u0;
    return Bnd{a.optr[pc], a.optr[pc + nuw]};
  };
  uint32_t ecol[RPW], eval[RPW];
  // the entry slots a pass needs: the wave's longest range over LPR lanes (wave-uniform)
  auto slots = [&](const Bnd& bd, int pass) __attribute__((always_inline)) -> int {
    int len = (int)min(min(bd.s1, a.ncap) - max(bd.s0, (int64_t)0) - (int64_t)64 * pass, (int64_t)64);
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) len = max(len, __shfl_xor(len, m));
    return __builtin_amdgcn_readfirstlane(min(max(len, 0) + LPR - 1, 64) / LPR);
  };
  // entries start + 64 pass + lr_ + LPR i, i < ns, of the lane's range (indices clamped to the capacity)
  auto load_entries = [&](const Bnd& bd, int pass, int ns) __attribute__((always_inline)) {
    const int64_t s0 = max(bd.s0, (int64_t)0) + 64 * pass + lr_;
#pragma unroll
    for (int i = 0; i < RPW; ++i) {
      if (i < ns) {  // (uniform)
        const int64_t k = min(s0 + LPR * i, a.ncap - 1);
        ecol[i] = reinterpret_cast<const uint32_t*>(a.ocol)[2 * k];  // the column's low dword
        eval[i] = a.oval[k];
      }
    }
  };
  auto scatter = [&](uint16_t* tb, const Bnd& bd, int pass, int ns) __attribute__((always_inline)) {
    const int64_t s0 = max(bd.s0, (int64_t)0) + 64 * pass + lr_, s1 = min(bd.s1, a.ncap);
    uint16_t* row = tb + rq * RSTR + pq * SEG;
#pragma unroll
    for (int i = 0; i < RPW; ++i) {
      if (i < ns) {  // (uniform)
        const int d = (int)ecol[i] - cbase;
        const bool ok = s0 + LPR * i < s1 && d >= 0 && d < nuw * G;
        uint16_t* dst = ok ? row + d : dummy + lane;
        *dst = (uint16_t)eval[i];
      }
    }
  };
  // the passes after the first, for ranges of more than 64 entries (rare), loaded and written in turn
  auto scatter_rest = [&](uint16_t* tb, const Bnd& bd) __attribute__((always_inline)) {
    const int64_t len = min(bd.s1, a.ncap) - max(bd.s0, (int64_t)0);
    for (int pass = 1; __builtin_amdgcn_ballot_w64(len > (int64_t)64 * pass) != 0; ++pass) {  // (uniform)
      const int ns = slots(bd, pass);
      load_entries(bd, pass, ns);
      scatter(tb, bd, pass, ns);
    }
  };
  // (the workers' 256 threads)
  auto zero_tile = [&](uint16_t* tb) __attribute__((always_inline)) {
    for (int i = (int)threadIdx.x - 256; i < TILE / 8; i += 256) *reinterpret_cast<u32x4*>(tb + 8 * i) = u32x4{0u, 0u, 0u, 0u};
  };

  const float zero[E] = {};
  constexpr float kHalf = (float)(1 << (BITS - 1));
  // x_hat of a block from tile tb (the lane's own 16 columns of every plane: outlier values in,
  // x_hat out): bf16(bf16(bf16((code - 2^(b-1)) s) + o) + bf16(l @ r)), as legacy_value
  auto compute = [&](const Blk& d, uint16_t* tb) __attribute__((always_inline)) {
    static_for<0, NP>([&](auto pc) {
      constexpr int p = decltype(pc)::value;
      float lr[E];
      residual_unit<G, K>(vop[p], d.lop, zero, lr);
      uint16_t* tp = tb + j * RSTR + p * SEG + w * G + E * g;
      u32x4 ov[2] = {u32x4{0u, 0u, 0u, 0u}, u32x4{0u, 0u, 0u, 0u}};
      if constexpr (COO) {
        ov[0] = *reinterpret_cast<const u32x4*>(tp);
        ov[1] = *reinterpret_cast<const u32x4*>(tp + 8);
      }
      u32x4 xo[2];
      const uint16_t* sp = stab + p * SEG + w * G + E * g;
      const u32x4 scp[2] = {*reinterpret_cast<const u32x4*>(sp), *reinterpret_cast<const u32x4*>(sp + 8)};
#pragma unroll
      for (int e = 0; e < E; e += 2) {
        const uint32_t sw = scp[e >> 3][(e >> 1) & 3], lp = pack_bf16x2(lr[e], lr[e + 1]);
        float av[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const uint32_t code = (d.cb[(e + h) >> 2] >> (8 * ((e + h) & 3) + BITS * p)) & kMask;
          const float s = h ? bf_hi(sw) : bf_lo(sw);
          av[h] = __builtin_fmaf((float)code, s, -kHalf * s);  // (code - 2^(b-1)) * s, exact in fp32
        }
        if constexpr (BITS > 2) {  // (already a bf16 value at 1 and 2 bits)
          const uint32_t ap = pack_bf16x2(av[0], av[1]);
          av[0] = bf_lo(ap);
          av[1] = bf_hi(ap);
        }
        if constexpr (COO) {
          const uint32_t ow = ov[e >> 3][(e >> 1) & 3];
          const uint32_t ap = pack_bf16x2(av[0] + bf_lo(ow), av[1] + bf_hi(ow));
          av[0] = bf_lo(ap);
          av[1] = bf_hi(ap);
        }
        xo[e >> 3][(e >> 1) & 3] = pack_bf16x2(av[0] + bf_lo(lp), av[1] + bf_hi(lp));
      }
      *reinterpret_cast<u32x4*>(tp) = xo[0];
      *reinterpret_cast<u32x4*>(tp + 8) = xo[1];
    });
  };
  // tile tb -> the rows of block i: 16 rows x NP planes x the units' 64 nuw columns (16 bytes a
  // lane; rows past M and blocks past the run fall outside the store range)
  auto store_tile = [&](const uint16_t* tb, int i) __attribute__((always_inline)) {
    const int rb = rb0 + min(i, nblk - 1);
    const uint32_t rows = i < nblk ? (uint32_t)min(16, M - rb * 16) : 0u;
    const __amdgpu_buffer_rsrc_t rs = uniform_rsrc(a.out + (bm0 + (int64_t)rb * 16) * N, rows * (uint32_t)N * 2u);
    constexpr int CH = SEG / 8;  // 16-byte chunks per (row, plane)
    static_assert((16 * NP * CH) % 256 == 0, "whole store passes");
#pragma unroll
    for (int c0 = 0; c0 < 16 * NP * CH; c0 += 256) {
      const int c = c0 + (int)threadIdx.x;
      const int r = c / (NP * CH), rem = c % (NP * CH), p = rem / CH, k = rem % CH;
      const u32x4 v = *reinterpret_cast<const u32x4*>(tb + r * RSTR + p * SEG + 8 * k);
      const uint32_t off = (uint32_t)((r * N + p * (int)NB + u0 * G + 8 * k) * 2);
      __builtin_amdgcn_raw_buffer_store_b128(v, rs, 8 * k < nuw * G ? off : 0x7ffffff0u, 0, 2);
    }
  };

  Blk ring[PD];
  const int npos = (nblk + PD - 1) / PD * PD;  // positions, whole ring rounds
  if constexpr (COO) {
    if (worker) {
      // block 0's entries into tile 0, block 1's requested; per position: zero the next tile
      // (between the barriers), then write the next block's entries into it and request those
      // of the block after
      const Bnd bnd0 = load_bounds(0);
      Bnd bnd_c = load_bounds(1), bnd_n = load_bounds(2), bnd_nn = load_bounds(3);
      zero_tile(lt);
      zero_tile(lt + TILE);
      int ns = slots(bnd0, 0);
      load_entries(bnd0, 0, ns);
      lds_barrier();  // B0: both tiles zeroed
      scatter(lt, bnd0, 0, ns);
      scatter_rest(lt, bnd0);
      int ns_c = slots(bnd_c, 0);
      load_entries(bnd_c, 0, ns_c);  // block 1's
#pragma unroll 1
      for (int bi = 0; bi < npos; ++bi) {
        uint16_t* tn = lt + ((bi + 1) & 1) * TILE;
        lds_barrier();  // B1: tn's previous rows have left
        zero_tile(tn);
        lds_barrier();  // B2: tn zeroed
        scatter(tn, bnd_c, 0, ns_c);  // block bi + 1
        scatter_rest(tn, bnd_c);
        bnd_c = bnd_n;
        bnd_n = bnd_nn;
        ns_c = slots(bnd_c, 0);
        load_entries(bnd_c, 0, ns_c);  // block bi + 2
        bnd_nn = load_bounds(bi + 4);
      }
    } else {
      static_for<0, PD>([&](auto kc) { load_blk(decltype(kc)::value, ring[decltype(kc)::value]); });
      lds_barrier();  // B0
#pragma unroll 1
      for (int bb = 0; bb < npos; bb += PD)
        static_for<0, PD>([&](auto kc) {
          constexpr int k = decltype(kc)::value;
          const int bi = bb + k;
          uint16_t* tc = lt + (bi & 1) * TILE;
          lds_barrier();  // B1: block bi's outliers are in tc
          compute(ring[k], tc);
          lds_barrier();  // B2: x_hat of block bi in tc
          store_tile(tc, bi);
          __builtin_amdgcn_sched_barrier(0);
          load_blk(bi + PD, ring[k]);
          __builtin_amdgcn_sched_barrier(0);
        });
    }
  } else {
    static_for<0, PD>([&](auto kc) { load_blk(decltype(kc)::value, ring[decltype(kc)::value]); });
#pragma unroll 1
    for (int bb = 0; bb < npos; bb += PD)
      static_for<0, PD>([&](auto kc) {
        constexpr int k = decltype(kc)::value;
        const int bi = bb + k;
        uint16_t* tc = lt + (bi & 1) * TILE;
        lds_barrier();  // B1: tc's previous rows have left
        compute(ring[k], tc);
        lds_barrier();  // B2
        store_tile(tc, bi);
        __builtin_amdgcn_sched_barrier(0);
        load_blk(bi + PD, ring[k]);
        __builtin_amdgcn_sched_barrier(0);
      });
  }
}

// ------------------------------------------------------------------ dequant-GEMM
// out[b, m, c] = bf16( sum_n x_hat[b, m, n] * y[b, n, c] ), the sum in fp32, with x_hat the
// fused decode's value bf16(bf16(bf16((code - 2^(b-1)) * s) + bf16(l @ r))): the reference's
// triton_matmul_decompress (extraction_fuse_matmul.py:224-249, kernel :151-221) on the torch form
// of its decode.  x_hat never leaves the registers.
struct LegacyGemmArgs {
  const uint16_t* l;   // [M, K]
  const uint16_t* rt;  // [N, K]
  const uint8_t* q;    // [B, M, N/NP]
  const uint16_t* s;   // [s_rows, N]
  int64_t s_rows;
  const uint16_t* y;   // [B, N, ldy]: columns c0 .. c0 + NOUT - 1 for this launch (y points at c0)
  int64_t ldy;
  uint16_t* out;       // [B, M, ldo] (out points at column c0)
  int64_t ldo;
  int64_t M, N;
  int n_out;           // scalar path: output columns
};

// MFMA path (every plane a whole number of 64-column units).  Grid: B * ceil(row blocks / RB)
// workgroups of 8 waves; a workgroup owns RB 16-row blocks of one batch.  Work items are
// (unit, plane) pairs, unit-major, so the waves that run together share a unit's code rows in
// L2; wave w takes items w, w + 8, ...  An item's operands (rt and y rows of the plane's 64
// columns in the reconstruction layout, the lane's 16 scales, the RB blocks' code vectors) sit in
// one of two register slots, loaded while the other item is computed.  Per item the y operands are
// transposed once (identity MFMA); per row block the reconstruction MFMA gives bf16(l @ r) in the
// lane's 16 columns, the decode's roundings give x_hat, and x_hat (bf16, exact) is the B operand of
// the product MFMA.  The 8 waves' partial tiles are then summed through LDS in wave order.
template <int BITS, int K, int NOUT, int RB>
__global__ __launch_bounds__(512) void k_legacy_gemm(LegacyGemmArgs a) {
  constexpr int NP = 8 / BITS, G = 64, E = 16, RT = K / 16, TO = NOUT / 16, NW = 8;
  constexpr uint32_t kMask = BITS == 8 ? 0xffu : (1u << BITS) - 1u;
  __shared__ f32x4 part[NW][TO][64];
  const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int j = lane & 15, g = lane >> 4;
  const int M = (int)a.M, N = (int)a.N;
  const int nrb = (M + 15) / 16, gx = (nrb + RB - 1) / RB;
  const int b = blockIdx.x / gx;
  const int rb0 = (blockIdx.x - b * gx) * RB;
  const int nu = N / NP / G, ni = nu * NP;
  const int64_t NB = N / NP;
  const uint16_t* srow = a.s + (a.s_rows == 1 ? 0 : (int64_t)b * N);
  const uint16_t* yb = a.y + (int64_t)b * N * a.ldy;
  const uint8_t* qb = a.q + (int64_t)b * M * NB;
  const u32x2 ident = identity_bop(j, g);
  const float zero[E] = {};

  f32x4 acc[RB][TO];
  u32x2 lop[RB][RT];
#pragma unroll
  for (int i = 0; i < RB; ++i) {
    const int64_t row = min(min(rb0 + i, nrb - 1) * 16 + j, M - 1);
#pragma unroll
    for (int t = 0; t < TO; ++t) acc[i][t] = zero4();
#pragma unroll
    for (int t = 0; t < RT; ++t) lop[i][t] = ld8(a.l + row * K + 16 * t + 4 * g);
  }
  struct Item {
    u32x2 vop[G / 16][RT];  // rt rows of the item's columns (reconstruction A operand)
    u32x2 ya[G / 16][TO];   // y rows of the item's columns, same layout
    u32x4 sc[2];            // the lane's 16 scales (bf16)
    u32x4 cb[RB];           // the lane's 16 code bytes of each row block
  };
  auto load_item = [&](int it, Item& d) __attribute__((always_inline)) {
    const int u = it / NP, p = it % NP;
    const int base = unit_base(p, u, N, NP, G);
    load_vops<G, K>(a.rt, base, j, g, d.vop);
#pragma unroll
    for (int q = 0; q < G / 16; ++q)
#pragma unroll
      for (int t = 0; t < TO; ++t) d.ya[q][t] = ld8(yb + (int64_t)vrow_res<G>(base, j, q) * a.ldy + 16 * t + 4 * g);
    d.sc[0] = ld16(srow + base + E * g);
    d.sc[1] = ld16(srow + base + E * g + 8);
#pragma unroll
    for (int i = 0; i < RB; ++i) {
      const int64_t row = min(min(rb0 + i, nrb - 1) * 16 + j, M - 1);
      d.cb[i] = ld16_stream(qb + row * NB + u * G + E * g);
    }
  };
  // x_hat = bf16(a + bf16(l @ r)) with a = bf16((code - 2^(b-1)) * s), as legacy_value, two columns
  // at a time: (code - 2^(b-1)) * s is fma(code, s, -2^(b-1) s), exact in fp32 (an integer of at
  // most 8 bits times a bf16), and already a bf16 value for 1 and 2 bits (|code - 2^(b-1)| <= 2);
  // each bf16 rounding is one v_cvt_pk_bf16_f32 (round to nearest even, as bf16r) per pair, and
  // the last one leaves the pair packed as the product's operand.
  auto compute_item = [&](const Item& d, int p) __attribute__((always_inline)) {
    u32x4 yt[G / 32][TO];
    transpose_vops<G, NOUT>(d.ya, ident, yt);
    float sc[E], zb[E];
    unpack8(d.sc[0], sc);
    unpack8(d.sc[1], sc + 8);
#pragma unroll
    for (int e = 0; e < E; ++e) zb[e] = -(float)(1 << (BITS - 1)) * sc[e];
    const int sh = BITS * p;
#pragma unroll
    for (int i = 0; i < RB; ++i) {
      float lr[E];
      residual_unit<G, K>(d.vop, lop[i], zero, lr);
      u32x4 xb[G / 32];
#pragma unroll
      for (int e = 0; e < E; e += 2) {
        const uint32_t lp = pack_bf16x2(lr[e], lr[e + 1]);  // bf16(l @ r) of both columns
        float av[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const uint32_t code = (d.cb[i][(e + h) >> 2] >> (8 * ((e + h) & 3) + sh)) & kMask;
          av[h] = __builtin_fmaf((float)code, sc[e + h], zb[e + h]);
        }
        if constexpr (BITS > 2) {
          const uint32_t ap = pack_bf16x2(av[0], av[1]);
          av[0] = bf_lo(ap);
          av[1] = bf_hi(ap);
        }
        xb[e / 8][(e / 2) % 4] = pack_bf16x2(av[0] + bf_lo(lp), av[1] + bf_hi(lp));
      }
      project_unit_vt<G, NOUT>(yt, xb, acc[i]);
    }
  };
  // Items w, w + NW, ... through the two slots.  The loop body has no condition (a compute under
  // a branch made the compiler wait for every outstanding load, the other slot's included, at the
  // join); an odd last item runs after the loop.  NW is a multiple of NP, so every item of a wave
  // is in plane w % NP.
  static_assert(NW % NP == 0, "one plane per wave");
  const int nit = w < ni ? (ni - w + NW - 1) / NW : 0, pw = w % NP;
  Item ring[2];
#pragma unroll
  for (int sl = 0; sl < 2; ++sl) load_item(min(w + sl * NW, ni - 1), ring[sl]);
  int i0 = 0;
  for (; i0 + 1 < nit; i0 += 2) {
    compute_item(ring[0], pw);
    __builtin_amdgcn_sched_barrier(0);
    load_item(min(w + (i0 + 2) * NW, ni - 1), ring[0]);
    __builtin_amdgcn_sched_barrier(0);
    compute_item(ring[1], pw);
    __builtin_amdgcn_sched_barrier(0);
    load_item(min(w + (i0 + 3) * NW, ni - 1), ring[1]);
    __builtin_amdgcn_sched_barrier(0);
  }
  if (i0 < nit) compute_item(ring[0], pw);  // wave-uniform

  // acc[i][t] in lane (j, g), component v: out[row j][16t + 4g + v] (partial over this wave's items)
  constexpr int F = TO * 256 / NW, S = 64 / F, PPL = NW / S;
  static_assert(F >= 1 && F <= 64 && 64 % F == 0 && NW % S == 0, "out reduction split");
  const float* partf = reinterpret_cast<const float*>(&part[0][0][0]);
  uint16_t* ob = a.out + (int64_t)b * M * a.ldo;
#pragma unroll
  for (int i = 0; i < RB; ++i) {
    if (rb0 + i >= nrb) break;  // uniform
#pragma unroll
    for (int t = 0; t < TO; ++t) part[w][t][lane] = acc[i][t];
    __syncthreads();
    const int f = lane % F, pg = lane / F;
    const int fi = w * F + f;
    const int t = fi >> 8, src = (fi >> 2) & 63, v = fi & 3;
    float s = 0.f;
#pragma unroll
    for (int k = 0; k < PPL; ++k) s += partf[(((pg * PPL + k) * TO + t) * 64 + src) * 4 + v];
#pragma unroll
    for (int m = F; m < 64; m <<= 1) s += __shfl_xor(s, m);
    const int row = (rb0 + i) * 16 + (src & 15);
    const int col = 16 * t + 4 * (src >> 4) + v;
    if (pg == 0 && row < M) ob[(int64_t)row * a.ldo + col] = (uint16_t)pack_bf16x2(s, 0.f);
    __syncthreads();
  }
}

// Scalar path (any shape): one workgroup per row (b, m); thread t decodes columns t, t + 256, ...
// (l @ r in fp64, exact, as k_legacy_scalar) and multiplies them into up to 32 fp32 sums; the 256
// threads' sums are added through LDS in thread order.  Output columns in chunks of 32.
template <int BITS>
__global__ __launch_bounds__(256) void k_legacy_gemm_scalar(LegacyGemmArgs a, int K) {
  constexpr int NP = 8 / BITS, OC = 32;
  constexpr uint32_t kMask = BITS == 8 ? 0xffu : (1u << BITS) - 1u;
  __shared__ float red[OC][257];
  const int64_t M = a.M, N = a.N, NB = N / NP;
  const int64_t bm = blockIdx.x, b = bm / M, m = bm - b * M;
  const uint16_t* srow = a.s + (a.s_rows == 1 ? 0 : b * N);
  const uint16_t* lrow = a.l + m * K;
  const uint16_t* yb = a.y + b * N * a.ldy;
  const int t = threadIdx.x;
  for (int o0 = 0; o0 < a.n_out; o0 += OC) {
    const int nc = min(OC, a.n_out - o0);
    float acc[OC];
#pragma unroll
    for (int o = 0; o < OC; ++o) acc[o] = 0.f;
    for (int64_t col = t; col < N; col += 256) {
      const int64_t c = col % NB;
      const int p = (int)(col / NB);
      const uint16_t* rrow = a.rt + col * K;
      double dot = 0.0;
      for (int k = 0; k < K; ++k)
        dot = __builtin_fma((double)__uint_as_float((uint32_t)lrow[k] << 16),
                            (double)__uint_as_float((uint32_t)rrow[k] << 16), dot);
      const uint32_t code = ((uint32_t)a.q[bm * NB + c] >> (BITS * p)) & kMask;
      const float sc = __uint_as_float((uint32_t)srow[col] << 16);
      const float xh = legacy_value<BITS, false>(code, sc, 0.f, bf16r((float)dot));
      const uint16_t* yr = yb + col * a.ldy + o0;
#pragma unroll
      for (int o = 0; o < OC; ++o)
        if (o < nc) acc[o] = __builtin_fmaf(xh, __uint_as_float((uint32_t)yr[o] << 16), acc[o]);
    }
#pragma unroll
    for (int o = 0; o < OC; ++o) red[o][t] = acc[o];
    __syncthreads();
    if (t < nc) {
      float s = 0.f;
      for (int i = 0; i < 256; ++i) s += red[t][i];
      a.out[bm * a.ldo + o0 + t] = (uint16_t)pack_bf16x2(s, 0.f);
    }
    __syncthreads();
  }
}

// Scalar form of the hist pass: one thread per column of one row (any shape).
__global__ __launch_bounds__(256) void k_hist_scalar(LegacyArgs a, int K, int64_t chunks) {
  __shared__ uint32_t lh[256];
  lh[threadIdx.x] = 0u;
  const int64_t sel = a.sel[0];
  __syncthreads();
  const int64_t m = blockIdx.x / chunks;
  const int64_t c = (blockIdx.x - m * chunks) * 256 + threadIdx.x;
  if (c < a.N) {
    const uint16_t* lrow = a.l + m * K;
    const uint16_t* rrow = a.rt + c * K;
    double acc = 0.0;
    for (int k = 0; k < K; ++k)
      acc = __builtin_fma((double)__uint_as_float((uint32_t)lrow[k] << 16),
                          (double)__uint_as_float((uint32_t)rrow[k] << 16), acc);
    const float xv = __uint_as_float((uint32_t)a.x[m * a.ldx_m + c] << 16);
    const int bin = hist_bin(bf16r(xv - bf16r((float)acc)), sel);
    if (bin >= 0) atomicAdd(&lh[bin], 1u);
  }
  __syncthreads();
  if (lh[threadIdx.x] != 0u) atomicAdd(&a.hist[threadIdx.x], lh[threadIdx.x]);
}

// hist[0..255] = 0, sel = {-1, k}.
__global__ __launch_bounds__(256) void k_kth_init(uint32_t* __restrict__ hist, int64_t* __restrict__ sel, int64_t k) {
  hist[threadIdx.x] = 0u;
  if (threadIdx.x == 0) {
    sel[0] = -1;
    sel[1] = k;
  }
}

// The bin holding the sel[1]-th smallest key (1-based) of the histogram.  First pass: sel =
// {bin, rank within it}, histogram cleared for the second pass.  Second pass (fine): the key
// (sel[0] << 7 | bin) as an fp32 value in out.  256 threads, one bin each.
__global__ __launch_bounds__(256) void k_kth_select(uint32_t* __restrict__ hist, int64_t* __restrict__ sel, int fine,
                                                    float* __restrict__ out) {
  __shared__ uint64_t wsum[4];
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  const uint64_t h = (fine && t >= 128) ? 0u : hist[t];
  const uint64_t k = (uint64_t)sel[1];
  uint64_t incl = h;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const uint64_t o = __shfl_up(incl, d);
    if (lane >= d) incl += o;
  }
  if (lane == 63) wsum[w] = incl;
  __syncthreads();
  for (int i = 0; i < w; ++i) incl += wsum[i];
  const int64_t prev = sel[0];
  __syncthreads();  // every thread has read sel before it is rewritten
  if (incl >= k && incl - h < k) {  // exactly one bin: the cumulative count first reaches k
    if (!fine) {
      sel[0] = t;
      sel[1] = (int64_t)(k - (incl - h));
    } else {
      out[0] = __uint_as_float((uint32_t)((prev << 7) | t) << 16);
    }
  }
  hist[t] = 0u;
}

// ------------------------------------------------------------------ host side
// 64-row blocks per workgroup of the MFMA path: 4, or 2 / 1 where 4 would give fewer than two
// workgroups per CU (small M or few units: the reference speed tests' M = 512 gives 8).
static int legacy_rows_per_wg(int64_t M, int64_t wg_cols) {
  const int64_t want = 2 * (int64_t)cu_count();
  for (int rb = 4; rb > 1; rb /= 2)
    if ((M + 64 * rb - 1) / (64 * rb) * wg_cols >= want) return rb;
  return 1;
}

// The row-tile decode (k_legacy_rows) for decodes without dense outliers at 2, 4 and 8 bits,
// when every workgroup of 4 units has whole units and there are enough blocks for about two
// workgroups per CU (smaller shapes keep k_legacy_mfma, which splits rows more finely); runs of
// whole ring rounds (PD blocks).  Returns false where it does not apply.
template <int MODE, int BITS, int OSRC>
static bool legacy_rows_launch(const LegacyArgs& a, int K, int64_t B, hipStream_t st, int* status) {
  if constexpr (MODE != kDecode || OSRC == 1 || BITS == 1) {
    return false;
  } else {
    using Lr = LegacyRows<BITS>;
    const int64_t NB = a.N / Lr::NP, nu = NB / 64, nrb = (a.M + 15) / 16;
    if (NB % 64 != 0 || nu < Lr::NW || 16 * a.N * 2 >= ((int64_t)1 << 31)) return false;
    const int64_t ug = (nu + Lr::NW - 1) / Lr::NW, tiles = B * ug;
    const int64_t want = 2 * (int64_t)cu_count();
    if (tiles * nrb < want * 2 * Lr::PD) return false;  // under two ring rounds per workgroup
    int64_t runs = std::max<int64_t>(1, want / tiles);
    int64_t rbw = (nrb + runs - 1) / runs;
    rbw = (rbw + Lr::PD - 1) / Lr::PD * Lr::PD;
    runs = (nrb + rbw - 1) / rbw;
    const int64_t nwg = tiles * runs;
    if (nwg > INT32_MAX) return false;
    const bool coo = OSRC != 0 && a.ncap > 0;
    auto go = [&](auto kern) __attribute__((always_inline)) {
      (void)hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)Lr::LDS);
      *status = launch(kern, dim3((unsigned)nwg), dim3(coo ? 512 : 256), Lr::LDS, st, a, (int)rbw, (int)ug);
    };
    if (K == 16) {
      if (coo) go(k_legacy_rows<BITS, 16, true>);
      else go(k_legacy_rows<BITS, 16, false>);
    } else {
      if (coo) go(k_legacy_rows<BITS, 32, true>);
      else go(k_legacy_rows<BITS, 32, false>);
    }
    return true;
  }
}

template <int MODE, int BITS, int OSRC>
static int legacy_launch(const LegacyArgs& a, int K, int64_t B, bool mfma_ok, hipStream_t st) {
  constexpr int NP = (MODE == kAdd) ? 1 : 8 / BITS;
  if (mfma_ok) {
    int status = LRQ_OK;
    if (legacy_rows_launch<MODE, BITS, OSRC>(a, K, B, st, &status)) return status;
  }
  const int64_t NB = a.N / NP;
  const int rb = legacy_rows_per_wg(a.M, NB / 64 * B);
  const int64_t nwg = (a.M + 64 * rb - 1) / (64 * rb) * (NB / 64) * B;
  if (mfma_ok && NB % 64 == 0 && nwg <= INT32_MAX) {
    // 4 row blocks per workgroup, fewer where that would leave under two workgroups per CU
    LegacyArgs la = a;
    la.rb = rb;
    const dim3 grid((unsigned)nwg);
    if (K == 16) LRQ_TRY(launch((k_legacy_mfma<MODE, BITS, 16, OSRC>), grid, dim3(256), 0, st, la));
    else LRQ_TRY(launch((k_legacy_mfma<MODE, BITS, 32, OSRC>), grid, dim3(256), 0, st, la));
  } else {
    const int64_t chunks = (NB + 255) / 256;
    if (B * a.M * chunks > INT32_MAX) return LRQ_ERR_SHAPE;
    LRQ_TRY(launch((k_legacy_scalar<MODE, BITS, OSRC>), dim3((unsigned)(B * a.M * chunks)), dim3(256), 0, st, a,
                       K, chunks));
  }
  return LRQ_OK;
}

template <int MODE, int OSRC>
static int legacy_bits(const LegacyArgs& a, int K, int64_t B, int bits, bool mfma_ok, hipStream_t st) {
  switch (bits) {
    case 1: return legacy_launch<MODE, 1, OSRC>(a, K, B, mfma_ok, st);
    case 2: return legacy_launch<MODE, 2, OSRC>(a, K, B, mfma_ok, st);
    case 4: return legacy_launch<MODE, 4, OSRC>(a, K, B, mfma_ok, st);
    case 8: return legacy_launch<MODE, 8, OSRC>(a, K, B, mfma_ok, st);
    default: return LRQ_ERR_UNSUPPORTED;
  }
}

// Shape / argument checks common to every legacy entry point.
static int legacy_check(const void* l, const void* rt, int32_t K, int64_t B, int64_t M, int64_t N, int32_t bits,
                        const void* s, int64_t s_rows, bool need_s) {
  if (l == nullptr || rt == nullptr) return LRQ_ERR_NULL;
  if (need_s && s == nullptr) return LRQ_ERR_NULL;
  if (K != 16 && K != 32) return LRQ_ERR_UNSUPPORTED;
  if (bits != 1 && bits != 2 && bits != 4 && bits != 8) return LRQ_ERR_UNSUPPORTED;
  if (B < 0 || M < 0 || N <= 0 || M > INT32_MAX || N > INT32_MAX) return LRQ_ERR_SHAPE;
  if (N % (8 / bits) != 0) return LRQ_ERR_SHAPE;
  if (need_s && s_rows != 1 && s_rows != B) return LRQ_ERR_SHAPE;
  if (!aligned(l, 2) || !aligned(rt, 2) || (need_s && !aligned(s, 2))) return LRQ_ERR_ALIGN;
  return LRQ_OK;
}

// The MFMA path reads and writes 16-byte vectors and 8-byte L / V operands.
static bool vec_ok(std::initializer_list<const void*> ptrs) {
  for (const void* p : ptrs)
    if (p != nullptr && !aligned(p, 16)) return false;
  return true;
}

}  // namespace lrq

using namespace lrq;

extern "C" int lrq_legacy_encode(const void* l, const void* rt, int32_t K, const void* x, int64_t B, int64_t M,
                                 int64_t N, int64_t ldx_b, int64_t ldx_m, const void* s, int64_t s_rows,
                                 int32_t bits, float outlier, void* o, void* q, void* stream) {
  int st = legacy_check(l, rt, K, B, M, N, bits, s, s_rows, true);
  if (st) return st;
  if (x == nullptr || o == nullptr || q == nullptr) return LRQ_ERR_NULL;
  if (ldx_m < N || (M > 1 && B > 1 && ldx_b < ldx_m * (M - 1) + N)) return LRQ_ERR_SHAPE;
  if (!aligned(x, 2) || !aligned(o, 2)) return LRQ_ERR_ALIGN;
  if (B == 0 || M == 0) return LRQ_OK;
  LegacyArgs a{};
  a.l = (const uint16_t*)l, a.rt = (const uint16_t*)rt, a.x = (const uint16_t*)x, a.ldx_b = ldx_b, a.ldx_m = ldx_m;
  a.s = (const uint16_t*)s, a.s_rows = s_rows, a.oout = (uint16_t*)o, a.qout = (uint8_t*)q, a.M = M, a.N = N;
  a.tau = bf16_value_host(bf16_bits_host(outlier));
  const bool mfma_ok = vec_ok({l, rt, x, s, o, q}) && ldx_b % 8 == 0 && ldx_m % 8 == 0 && N % 8 == 0;
  return legacy_bits<kEncode, 0>(a, K, B, bits, mfma_ok, (hipStream_t)stream);
}

// lrq_legacy_encode whose outlier compaction starts from the staged piece records the encode
// writes (the MFMA path: each 64-column piece's count and first entries, its dense values only
// when it has more entries than a record holds), so the dense outliers are neither written nor
// read whole; other shapes take the encode and the full compaction.
extern "C" int lrq_legacy_encode_coo(const void* l, const void* rt, int32_t K, const void* x, int64_t B, int64_t M,
                                     int64_t N, int64_t ldx_b, int64_t ldx_m, const void* s, int64_t s_rows,
                                     int32_t bits, float outlier, void* o, void* q, int64_t* indices, int64_t ld_idx,
                                     void* values, int64_t cap, int64_t* nnz, int64_t* piece_ptr, void* workspace,
                                     int64_t workspace_bytes, void* stream) {
  int st = legacy_check(l, rt, K, B, M, N, bits, s, s_rows, true);
  if (st) return st;
  if (x == nullptr || o == nullptr || q == nullptr) return LRQ_ERR_NULL;
  if (ldx_m < N || (M > 1 && B > 1 && ldx_b < ldx_m * (M - 1) + N)) return LRQ_ERR_SHAPE;
  if (!aligned(x, 2) || !aligned(o, 2)) return LRQ_ERR_ALIGN;
  st = coo_compact_check(o, B, M, N, indices, ld_idx, values, cap, nnz, piece_ptr, workspace, workspace_bytes);
  if (st) return st;
  const int NP = 8 / bits;
  const bool mfma_ok = vec_ok({l, rt, x, s, o, q}) && ldx_b % 8 == 0 && ldx_m % 8 == 0 && N % 8 == 0;
  const int64_t NB = N / NP;
  const float tau = bf16_value_host(bf16_bits_host(outlier));
  // (with tau >= 0 an element's |xr| > tau is exactly "an entry"; a negative threshold keeps every
  // element but the +-0 ones, counted by the compaction's own pass)
  const bool counted = mfma_ok && NB % 64 == 0 && NB / 64 <= 65535 && B <= 65535 && aligned(o, 16) && tau >= 0.f;
  if (!counted || B == 0 || M == 0) {
    LRQ_TRY(lrq_legacy_encode(l, rt, K, x, B, M, N, ldx_b, ldx_m, s, s_rows, bits, outlier, o, q, stream));
    return lrq_coo_compact(o, B, M, N, indices, ld_idx, values, cap, nnz, piece_ptr, workspace, workspace_bytes,
                           stream);
  }
  LegacyArgs a{};
  a.l = (const uint16_t*)l, a.rt = (const uint16_t*)rt, a.x = (const uint16_t*)x, a.ldx_b = ldx_b, a.ldx_m = ldx_m;
  a.s = (const uint16_t*)s, a.s_rows = s_rows, a.oout = (uint16_t*)o, a.qout = (uint8_t*)q, a.M = M, a.N = N;
  a.tau = tau;
  a.npc = (N + 63) / 64, a.pcnt = piece_ptr;
  LRQ_TRY((legacy_bits<kEncode, 1>(a, K, B, bits, true, (hipStream_t)stream)));
  return coo_compact_staged(o, B, M, N, indices, ld_idx, values, cap, nnz, piece_ptr, workspace, (hipStream_t)stream);
}

extern "C" int lrq_legacy_decode(const void* l, const void* rt, int32_t K, const void* q, const void* o,
                                 const void* s, int64_t s_rows, int64_t B, int64_t M, int64_t N, int32_t bits,
                                 void* out, void* stream) {
  int st = legacy_check(l, rt, K, B, M, N, bits, s, s_rows, true);
  if (st) return st;
  if (q == nullptr || out == nullptr) return LRQ_ERR_NULL;
  if (!aligned(out, 2) || (o != nullptr && !aligned(o, 2))) return LRQ_ERR_ALIGN;
  if (B == 0 || M == 0) return LRQ_OK;
  LegacyArgs a{};
  a.l = (const uint16_t*)l, a.rt = (const uint16_t*)rt, a.s = (const uint16_t*)s, a.s_rows = s_rows;
  a.qin = (const uint8_t*)q, a.oin = (const uint16_t*)o, a.out = (uint16_t*)out, a.M = M, a.N = N;
  const bool mfma_ok = vec_ok({l, rt, q, o, s, out}) && N % 8 == 0;
  if (o != nullptr) return legacy_bits<kDecode, 1>(a, K, B, bits, mfma_ok, (hipStream_t)stream);
  return legacy_bits<kDecode, 0>(a, K, B, bits, mfma_ok, (hipStream_t)stream);
}

extern "C" int lrq_legacy_fused(const void* l, const void* rt, int32_t K, const void* q, const void* s,
                                int64_t s_rows, int64_t B, int64_t M, int64_t N, int32_t bits, int32_t op,
                                const void* y, void* out, void* stream) {
  int st = legacy_check(l, rt, K, B, M, N, bits, s, s_rows, true);
  if (st) return st;
  if (op < 0 || op > 2) return LRQ_ERR_UNSUPPORTED;
  if (q == nullptr || out == nullptr || (op != 0 && y == nullptr)) return LRQ_ERR_NULL;
  if (!aligned(out, 2) || (y != nullptr && !aligned(y, 2))) return LRQ_ERR_ALIGN;
  if (B == 0 || M == 0) return LRQ_OK;
  LegacyArgs a{};
  a.l = (const uint16_t*)l, a.rt = (const uint16_t*)rt, a.s = (const uint16_t*)s, a.s_rows = s_rows;
  a.qin = (const uint8_t*)q, a.y = (const uint16_t*)y, a.out = (uint16_t*)out, a.M = M, a.N = N;
  const bool mfma_ok = vec_ok({l, rt, q, s, y, out}) && N % 8 == 0;
  hipStream_t hs = (hipStream_t)stream;
  switch (op) {
    case 0: return legacy_bits<kFusedStore, 0>(a, K, B, bits, mfma_ok, hs);
    case 1: return legacy_bits<kFusedSilu, 0>(a, K, B, bits, mfma_ok, hs);
    default: return legacy_bits<kFusedMul, 0>(a, K, B, bits, mfma_ok, hs);
  }
}

namespace lrq {
template <int BITS, int K, int NOUT>
static int legacy_gemm_chunk(const LegacyGemmArgs& a, int64_t B, hipStream_t st) {
  // 16-row blocks per workgroup: 4, or 2 / 1 where 4 would leave CUs without a workgroup
  const int64_t nrb = (a.M + 15) / 16, cu = cu_count();
  auto launch_rb = [&](auto rb) __attribute__((always_inline)) {
    constexpr int RB = decltype(rb)::value;
    const int64_t nwg = B * ((nrb + RB - 1) / RB);
    if (nwg > INT32_MAX) return (int)LRQ_ERR_SHAPE;
    return launch((k_legacy_gemm<BITS, K, NOUT, RB>), dim3((unsigned)nwg), dim3(512), 0, st, a);
  };
  if (B * ((nrb + 3) / 4) >= cu) return launch_rb(std::integral_constant<int, 4>{});
  if (B * ((nrb + 1) / 2) >= cu) return launch_rb(std::integral_constant<int, 2>{});
  return launch_rb(std::integral_constant<int, 1>{});
}

template <int BITS>
static int legacy_gemm_bits(LegacyGemmArgs a, int K, int64_t B, bool mfma_ok, hipStream_t st) {
  if (!mfma_ok) {
    if (B * a.M > INT32_MAX) return LRQ_ERR_SHAPE;
    return launch(k_legacy_gemm_scalar<BITS>, dim3((unsigned)(B * a.M)), dim3(256), 0, st, a, K);
  }
  // output columns in chunks of 32 (then 16); each chunk is one pass over the codes
  const uint16_t* y0 = a.y;
  uint16_t* o0 = a.out;
  for (int c0 = 0; c0 < a.n_out;) {
    const int nc = a.n_out - c0 >= 32 ? 32 : 16;
    a.y = y0 + c0;
    a.out = o0 + c0;
    int r;
    if (K == 16) r = nc == 32 ? legacy_gemm_chunk<BITS, 16, 32>(a, B, st) : legacy_gemm_chunk<BITS, 16, 16>(a, B, st);
    else r = nc == 32 ? legacy_gemm_chunk<BITS, 32, 32>(a, B, st) : legacy_gemm_chunk<BITS, 32, 16>(a, B, st);
    LRQ_TRY(r);
    c0 += nc;
  }
  return LRQ_OK;
}
}  // namespace lrq

extern "C" int lrq_legacy_dequant_gemm(const void* l, const void* rt, int32_t K, const void* q, const void* s,
                                       int64_t s_rows, int64_t B, int64_t M, int64_t N, int32_t bits, const void* y,
                                       int64_t ldy, int32_t n_out, void* out, int64_t ldo, void* stream) {
  int st = legacy_check(l, rt, K, B, M, N, bits, s, s_rows, true);
  if (st) return st;
  if (q == nullptr || y == nullptr || out == nullptr) return LRQ_ERR_NULL;
  if (n_out < 1 || ldy < n_out || ldo < n_out) return LRQ_ERR_SHAPE;
  if (!aligned(y, 2) || !aligned(out, 2)) return LRQ_ERR_ALIGN;
  if (B == 0 || M == 0) return LRQ_OK;
  LegacyGemmArgs a{};
  a.l = (const uint16_t*)l, a.rt = (const uint16_t*)rt, a.q = (const uint8_t*)q, a.s = (const uint16_t*)s;
  a.s_rows = s_rows, a.y = (const uint16_t*)y, a.ldy = ldy, a.out = (uint16_t*)out, a.ldo = ldo, a.M = M, a.N = N;
  a.n_out = n_out;
  const int64_t NB = N / (8 / bits);
  const bool mfma_ok = vec_ok({l, rt, q, s}) && NB % 64 == 0 && n_out % 16 == 0 && aligned(y, 8) && ldy % 4 == 0;
  hipStream_t hs = (hipStream_t)stream;
  switch (bits) {
    case 1: return legacy_gemm_bits<1>(a, K, B, mfma_ok, hs);
    case 2: return legacy_gemm_bits<2>(a, K, B, mfma_ok, hs);
    case 4: return legacy_gemm_bits<4>(a, K, B, mfma_ok, hs);
    default: return legacy_gemm_bits<8>(a, K, B, mfma_ok, hs);
  }
}

extern "C" int lrq_lowrank_add(const void* l, const void* rt, int32_t K, const void* x, int64_t B, int64_t M,
                               int64_t N, void* out, void* stream) {
  int st = legacy_check(l, rt, K, B, M, N, 8, nullptr, 1, false);
  if (st) return st;
  if (x == nullptr || out == nullptr) return LRQ_ERR_NULL;
  if (!aligned(x, 2) || !aligned(out, 2)) return LRQ_ERR_ALIGN;
  if (B == 0 || M == 0) return LRQ_OK;
  LegacyArgs a{};
  a.l = (const uint16_t*)l, a.rt = (const uint16_t*)rt, a.x = (const uint16_t*)x, a.ldx_b = M * N, a.ldx_m = N;
  a.out = (uint16_t*)out, a.M = M, a.N = N;
  const bool mfma_ok = vec_ok({l, rt, x, out}) && N % 8 == 0;
  return legacy_launch<kAdd, 8, 0>(a, K, B, mfma_ok, (hipStream_t)stream);
}

extern "C" int lrq_legacy_decode_coo(const void* l, const void* rt, int32_t K, const void* q, const int64_t* piece_ptr,
                                     const int64_t* cols, const void* vals, int64_t n_entries, const void* s,
                                     int64_t s_rows, int64_t B, int64_t M, int64_t N, int32_t bits, void* out,
                                     void* stream) {
  int st = legacy_check(l, rt, K, B, M, N, bits, s, s_rows, true);
  if (st) return st;
  if (q == nullptr || out == nullptr || piece_ptr == nullptr) return LRQ_ERR_NULL;
  if (n_entries < 0) return LRQ_ERR_SHAPE;
  if (n_entries > 0 && (cols == nullptr || vals == nullptr)) return LRQ_ERR_NULL;
  if (!aligned(out, 2) || !aligned(piece_ptr, 8) || !aligned(cols, 8) || !aligned(vals, 2)) return LRQ_ERR_ALIGN;
  if (B == 0 || M == 0) return LRQ_OK;
  LegacyArgs a{};
  a.l = (const uint16_t*)l, a.rt = (const uint16_t*)rt, a.s = (const uint16_t*)s, a.s_rows = s_rows;
  a.qin = (const uint8_t*)q, a.out = (uint16_t*)out, a.M = M, a.N = N;
  a.optr = piece_ptr, a.ocol = cols, a.oval = (const uint16_t*)vals, a.npc = (N + 63) / 64, a.ncap = n_entries;
  const bool mfma_ok = vec_ok({l, rt, q, s, out}) && N % 8 == 0;
  // more than about 4 entries per 64-column piece (1/16 of the elements): the wave gathers its
  // pieces' entries cooperatively (an LDS tile); sparser: each lane reads its piece's few entries
  if (mfma_ok && n_entries * 16 > B * M * N) return legacy_bits<kDecode, 3>(a, K, B, bits, mfma_ok, (hipStream_t)stream);
  return legacy_bits<kDecode, 2>(a, K, B, bits, mfma_ok, (hipStream_t)stream);
}

extern "C" int lrq_legacy_kth_residual(const void* l, const void* rt, int32_t K, const void* x, int64_t M, int64_t N,
                                       int64_t ldx_m, int64_t k, float* out, void* workspace, int64_t workspace_bytes,
                                       void* stream) {
  int st = legacy_check(l, rt, K, 1, M, N, 8, nullptr, 1, false);
  if (st) return st;
  if (x == nullptr || out == nullptr || workspace == nullptr) return LRQ_ERR_NULL;
  if (ldx_m < N) return LRQ_ERR_SHAPE;
  if (M * N >= ((int64_t)1 << 32) || k < 1 || k > M * N) return LRQ_ERR_SHAPE;
  if (workspace_bytes < 2048) return LRQ_ERR_WORKSPACE;
  if (!aligned(x, 2) || !aligned(out, 4) || !aligned(workspace, 16)) return LRQ_ERR_ALIGN;
  hipStream_t hs = (hipStream_t)stream;
  uint32_t* hist = reinterpret_cast<uint32_t*>(workspace);
  int64_t* sel = reinterpret_cast<int64_t*>(hist + 256);
  LegacyArgs a{};
  a.l = (const uint16_t*)l, a.rt = (const uint16_t*)rt, a.x = (const uint16_t*)x, a.ldx_b = 0, a.ldx_m = ldx_m;
  a.M = M, a.N = N, a.hist = hist, a.sel = sel;
  const bool mfma_ok = vec_ok({l, rt, x}) && ldx_m % 8 == 0 && N % 64 == 0;
  LRQ_TRY(launch(k_kth_init, dim3(1), dim3(256), 0, hs, hist, sel, k));
  for (int fine = 0; fine < 2; ++fine) {
    if (mfma_ok) {
      a.rb = legacy_rows_per_wg(M, N / 64);
      const dim3 grid((unsigned)((M + 64 * a.rb - 1) / (64 * a.rb) * (N / 64)));  // < 2^26 (M * N < 2^32)
      if (K == 16) LRQ_TRY(launch((k_legacy_mfma<kHist, 8, 16, 0>), grid, dim3(256), 0, hs, a));
      else LRQ_TRY(launch((k_legacy_mfma<kHist, 8, 32, 0>), grid, dim3(256), 0, hs, a));
    } else {
      const int64_t chunks = (N + 255) / 256;
      if (M * chunks > INT32_MAX) return LRQ_ERR_SHAPE;
      LRQ_TRY(launch(k_hist_scalar, dim3((unsigned)(M * chunks)), dim3(256), 0, hs, a, (int)K, chunks));
    }
    LRQ_TRY(launch(k_kth_select, dim3(1), dim3(256), 0, hs, hist, sel, fine, out));
  }
  return LRQ_OK;
}
