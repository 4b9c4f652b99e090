// Consumers that reduce along the hidden dimension, decompressing in-kernel:
//
//   k_softmax_bwd   dS = P (dP - rowsum(dP P)), P = bf16(decode(c)), one pass: the workgroup
//                   holds whole rows, so the row sum is finished in LDS between the
//                   reconstruction and the output (softmax_backward.py:6-7 formula; the
//                   reference has only the uncompressed triton_softmax_backward, :45-61).
//   k_dequant_gemm  out = bf16(decode(c)) @ A, A [N, n] bf16, fp32 accumulate on MFMA
//                   (extraction_fuse_matmul.py:224-249 intends this; its kernel reads wrong
//                   addresses, so the torch form :5-6 defines it).
//   k_dequant_gemm_t out = bf16(decode(c))^T @ G, G [M, n] bf16: the LoRA factor gradient
//                   x^T (dy B^T) (low_rank_system_profile_forward.py:14-18), a reduction over
//                   rows into per-row-group partials, then k_sum_parts.
//   k_softmax_rot, k_dequant_gemm_rotr, k_dequant_gemm_t_rot: the same on the rotated format,
//                   each rotating the 128-column blocks it rebuilds in registers (lrq_whtop.h).
#include "lrq_common.h"
#include "lrq_dequant.h"
#include "lrq_host.h"
#include "lrq_whtop.h"

#include <algorithm>
#include <mutex>

namespace lrq {

// ------------------------------------------------------------------ softmax backward
// Grid: ceil(row blocks / RBW); NW waves; wave w owns units w*UPW .. +UPW-1 and the host
// guarantees NW*UPW units per row.  Every input of the workgroup's RBW row blocks is
// requested up front (no load is issued after a store; see lrq_decode.hip).
template <int BITS, int G, int R, int NW, int UPW, int RBW>
__global__ __launch_bounds__(NW * 64) void k_softmax_bwd(
    const uint8_t* __restrict__ codes, int64_t ldc, const uint16_t* __restrict__ qparams, int64_t ldq,
    const uint16_t* __restrict__ Lin, int64_t ldl, const uint16_t* __restrict__ V, int M, int N,
    const uint16_t* __restrict__ dp, int64_t lddp, uint16_t* __restrict__ ds, int64_t ldds) {
  constexpr int NP = 8 / BITS, RT = R > 0 ? R / 16 : 1, E = G / 4;
  __shared__ float red[2][NW][16];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int j = lane & 15, g = lane >> 4;
  const int nrb = (M + 15) / 16;
  const int rb0 = blockIdx.x * RBW;

  u32x2 vop[UPW][NP][G / 16][RT];
  if constexpr (R > 0) {
#pragma unroll
    for (int uu = 0; uu < UPW; ++uu)
#pragma unroll
      for (int p = 0; p < NP; ++p) load_vops<G, R>(V, unit_base(p, w * UPW + uu, N, NP, G), j, g, vop[uu][p]);
  }
  struct In {
    u32x4 cb[UPW][G / 64];
    uint32_t qp[UPW][NP];
    u32x2 lop[RT];
    u32x4 d[UPW][NP][G / 32];
  };
  In in[RBW];
#pragma unroll
  for (int b = 0; b < RBW; ++b) {
    const int64_t row = min(min(rb0 + b, nrb - 1) * 16 + j, M - 1);
#pragma unroll
    for (int uu = 0; uu < UPW; ++uu) {
      const int u = w * UPW + uu;
#pragma unroll
      for (int i = 0; i < G / 64; ++i) in[b].cb[uu][i] = ld16_stream(codes + row * ldc + u * G + E * g + 16 * i);
      if constexpr (NP == 2) {
        const u32x2 q = ld8(qparams + row * ldq + u * 4);
        in[b].qp[uu][0] = q[0];
        in[b].qp[uu][1] = q[1];
      } else {
        in[b].qp[uu][0] = ld4(qparams + row * ldq + u * 2);
      }
#pragma unroll
      for (int p = 0; p < NP; ++p)
#pragma unroll
        for (int k = 0; k < G / 32; ++k)
          in[b].d[uu][p][k] = ld16_stream(dp + row * lddp + unit_base(p, u, N, NP, G) + E * g + 8 * k);
    }
    if constexpr (R > 0) {
#pragma unroll
      for (int t = 0; t < RT; ++t) in[b].lop[t] = ld8(Lin + row * ldl + 16 * t + 4 * g);
    }
  }
  __builtin_amdgcn_sched_barrier(0);

#pragma unroll
  for (int b = 0; b < RBW; ++b) {
    const int64_t row = min(min(rb0 + b, nrb - 1) * 16 + j, M - 1);
    float pv[UPW][NP][E];
    float part = 0.f;
#pragma unroll
    for (int uu = 0; uu < UPW; ++uu)
#pragma unroll
      for (int p = 0; p < NP; ++p) {
        reconstruct_plane<BITS, G, R>(in[b].cb[uu], in[b].qp[uu][p], p, vop[uu][p], in[b].lop, pv[uu][p]);
        float dv[E];
#pragma unroll
        for (int k = 0; k < G / 32; ++k) unpack8(in[b].d[uu][p][k], dv + 8 * k);
#pragma unroll
        for (int e = 0; e < E; e += 2) bf16_roundtrip2(pv[uu][p][e], pv[uu][p][e + 1]);
#pragma unroll
        for (int e = 0; e < E; ++e) part = __builtin_fmaf(pv[uu][p][e], dv[e], part);
      }
    // the row's four lanes, then the NW waves (through LDS)
    {
      float a = part, c = part;
      swap32(a, c);
      part = a + c;
      a = part, c = part;
      swap16(a, c);
      part = a + c;
    }
    if (g == 0) red[b & 1][w][j] = part;
    lds_barrier();
    float sum = 0.f;
#pragma unroll
    for (int w2 = 0; w2 < NW; ++w2) sum += red[b & 1][w2][j];
#pragma unroll
    for (int uu = 0; uu < UPW; ++uu)
#pragma unroll
      for (int p = 0; p < NP; ++p) {
        const int c0 = unit_base(p, w * UPW + uu, N, NP, G) + E * g;
        float dv[E], o[E];
#pragma unroll
        for (int k = 0; k < G / 32; ++k) unpack8(in[b].d[uu][p][k], dv + 8 * k);
#pragma unroll
        for (int e = 0; e < E; ++e) o[e] = pv[uu][p][e] * (dv[e] - sum);
#pragma unroll
        for (int k = 0; k < G / 32; ++k) st16(ds + row * ldds + c0 + 8 * k, pack8(o + 8 * k));
      }
  }
}

// Two-sweep softmax backward for rows of any number of units (rows too wide for one pass in
// a workgroup).  Grid: ceil(row blocks / RBW) workgroups of NW waves; wave w takes units
// w, w + NW, ... of the row.  Sweep 1 reconstructs P = bf16(decode) unit by unit and sums
// P * dP per row (quad swaps, then LDS across the waves); sweep 2 reconstructs P again and
// writes dS = P (dP - sum).  The row sum is taken in a fixed order (lane pairs, wave order),
// so dS does not depend on timing.  Rows past the end repeat the last row (identical stores).
//   HOLD > 0 (rows of NW .. NW*HOLD units, rank 0 or 16): every wave requests all of its units'
//            codes, qparams and dP of the row block at once and keeps them in registers for
//            both sweeps, so they are read once; the units' V operands are parked in the
//            wave's LDS slots at the start (operand order: one conflict-free 512-byte read
//            per operand) and read from there at each use.
//   HOLD = 0 (any width): each unit's inputs, V operands included, are requested one unit
//            ahead (a clamped repeat of the last unit at the end, so no load sits under a
//            branch) and read again in sweep 2.
template <int BITS, int G, int R, int NW, int HOLD>
struct Smx2s {
  static constexpr int NP = 8 / BITS, RT = R > 0 ? R / 16 : 1;
  static constexpr int VSLOT = NP * (G / 16) * RT * 64 * 8;  // one unit's V operands in LDS
  static constexpr size_t LDS = (HOLD > 0 && R > 0) ? (size_t)NW * HOLD * VSLOT : 0;
  static_assert(LDS <= 160 * 1024, "LDS budget");
};

template <int BITS, int G, int R, int NW, int HOLD>
__global__ __launch_bounds__(NW * 64) void k_softmax_2s(
    const uint8_t* __restrict__ codes, int64_t ldc, const uint16_t* __restrict__ qparams, int64_t ldq,
    const uint16_t* __restrict__ Lin, int64_t ldl, const uint16_t* __restrict__ V, int M, int N,
    const uint16_t* __restrict__ dp, int64_t lddp, uint16_t* __restrict__ ds, int64_t ldds, int RBW) {
  using Sm = Smx2s<BITS, G, R, NW, HOLD>;
  constexpr int NP = Sm::NP, RT = Sm::RT, E = G / 4;
  static_assert(HOLD == 0 || R <= 16, "held units keep one rank tile of V operands");
  __shared__ float red[NW][16];
  extern __shared__ __attribute__((aligned(16))) unsigned char vsm[];  // HOLD, R > 0: [NW][HOLD][VSLOT]
  const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int j = lane & 15, g = lane >> 4;
  const int nrb = (M + 15) / 16;
  const int units = N / (G * NP);
  const int nmine = (units - w + NW - 1) / NW;  // units of this wave (0 when units < NW and w >= units)
  struct In {
    u32x4 cb[G / 64];
    uint32_t qp[NP];
    u32x4 d[NP][G / 32];
  };
  using Vop = u32x2[NP][G / 16][RT];
  auto load = [&](In& in, int64_t row, int u) {
#pragma unroll
    for (int i = 0; i < G / 64; ++i) in.cb[i] = ld16_stream(codes + row * ldc + u * G + E * g + 16 * i);
    if constexpr (NP == 2) {
      const u32x2 q = ld8(qparams + row * ldq + u * 4);
      in.qp[0] = q[0];
      in.qp[1] = q[1];
    } else {
      in.qp[0] = ld4(qparams + row * ldq + u * 2);
    }
#pragma unroll
    for (int p = 0; p < NP; ++p)
#pragma unroll
      for (int k = 0; k < G / 32; ++k) {
        const uint16_t* a = dp + row * lddp + unit_base(p, u, N, NP, G) + E * g + 8 * k;
        in.d[p][k] = HOLD > 0 ? ld16_stream(a) : ld16(a);
      }
  };
  auto load_v = [&](Vop& v, int u) {
    if constexpr (R > 0) {
#pragma unroll
      for (int p = 0; p < NP; ++p) load_vops<G, R>(V, unit_base(p, u, N, NP, G), j, g, v[p]);
    }
  };
  // the LDS slot of held unit h of this wave; operand (p, q, t) is 64 lanes x 8 bytes
  auto vslot = [&](int h) { return reinterpret_cast<u32x2*>(vsm + ((size_t)w * HOLD + h) * Sm::VSLOT); };
  auto read_v = [&](Vop& v, int h) {
    if constexpr (R > 0) {
      const u32x2* sl = vslot(h);
#pragma unroll
      for (int p = 0; p < NP; ++p)
#pragma unroll
        for (int q = 0; q < G / 16; ++q)
#pragma unroll
          for (int t = 0; t < RT; ++t) v[p][q][t] = sl[((p * (G / 16) + q) * RT + t) * 64 + lane];
    }
  };
  // sweep 0: part += P * dP over the unit's lane columns; sweep 1: dS = P (dP - sum)
  auto work = [&](const In& cur, const Vop& v, int u, int sweep, const u32x2* lop, int64_t row, float& part,
                  float sum) {
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      float pv[E], dv[E];
      reconstruct_plane<BITS, G, R>(cur.cb, cur.qp[p], p, v[p], lop, pv);
#pragma unroll
      for (int k = 0; k < G / 32; ++k) unpack8(cur.d[p][k], dv + 8 * k);
#pragma unroll
      for (int e = 0; e < E; e += 2) bf16_roundtrip2(pv[e], pv[e + 1]);
      if (sweep == 0) {
#pragma unroll
        for (int e = 0; e < E; ++e) part = __builtin_fmaf(pv[e], dv[e], part);
      } else {
        float o[E];
#pragma unroll
        for (int e = 0; e < E; ++e) o[e] = pv[e] * (dv[e] - sum);
        const int c0 = unit_base(p, u, N, NP, G) + E * g;
#pragma unroll
        for (int k = 0; k < G / 32; ++k) st16(ds + row * ldds + c0 + 8 * k, pack8(o + 8 * k));
      }
    }
  };
  // the row's four lanes, then the NW waves in order (through LDS)
  auto row_sum = [&](float part) {
    float a = part, c = part;
    swap32(a, c);
    part = a + c;
    a = part, c = part;
    swap16(a, c);
    part = a + c;
    if (g == 0) red[w][j] = part;
    lds_barrier();
    float sum = 0.f;
#pragma unroll
    for (int w2 = 0; w2 < NW; ++w2) sum += red[w2][j];
    lds_barrier();  // every wave has read red before the next row block rewrites it
    return sum;
  };
  if constexpr (HOLD > 0 && R > 0) {
    // park this wave's V operands (the host launches this form only when 1 <= nmine <= HOLD);
    // a wave reads back only the slots it wrote, in order, so no barrier is needed
#pragma unroll
    for (int h = 0; h < HOLD; ++h) {
      if (h < nmine) {
        Vop v;
        load_v(v, w + h * NW);
        u32x2* sl = vslot(h);
#pragma unroll
        for (int p = 0; p < NP; ++p)
#pragma unroll
          for (int q = 0; q < G / 16; ++q)
#pragma unroll
            for (int t = 0; t < RT; ++t) sl[((p * (G / 16) + q) * RT + t) * 64 + lane] = v[p][q][t];
      }
    }
  }
  const int rb_end = min(nrb, (blockIdx.x + 1) * RBW);
#pragma unroll 1
  for (int rb = blockIdx.x * RBW; rb < rb_end; ++rb) {
    const int64_t row = min(rb * 16 + j, M - 1);
    u32x2 lop[RT];
    if constexpr (R > 0) {
#pragma unroll
      for (int t = 0; t < RT; ++t) lop[t] = ld8(Lin + row * ldl + 16 * t + 4 * g);
    }
    if constexpr (HOLD > 0) {
      In in[HOLD];
#pragma unroll
      for (int h = 0; h < HOLD; ++h) load(in[h], row, w + min(h, nmine - 1) * NW);
      float part = 0.f;
#pragma unroll
      for (int h = 0; h < HOLD; ++h) {
        if (h < nmine) {
          Vop v;
          read_v(v, h);
          work(in[h], v, w + h * NW, 0, lop, row, part, 0.f);
        }
      }
      const float sum = row_sum(part);
#pragma unroll
      for (int h = 0; h < HOLD; ++h) {
        if (h < nmine) {
          Vop v;
          read_v(v, h);
          work(in[h], v, w + h * NW, 1, lop, row, part, sum);
        }
      }
    } else {
      float part = 0.f, sum = 0.f;
#pragma unroll 1
      for (int sweep = 0; sweep < 2; ++sweep) {
        if (nmine > 0) {
          // units of 256 columns are loaded right before use (two in flight would spill)
          constexpr bool DB = G * NP <= 128;
          In in[DB ? 2 : 1];
          Vop v[DB ? 2 : 1];
          if constexpr (DB) {
            load(in[0], row, w);
            load_v(v[0], w);
          }
#pragma unroll 1
          for (int i = 0; i < nmine; i += 2) {
#pragma unroll
            for (int h = 0; h < 2; ++h) {
              if (i + h >= nmine) break;  // wave-uniform
              const int u = w + (i + h) * NW;
              if constexpr (DB) {
                const int un = w + min(i + h + 1, nmine - 1) * NW;
                load(in[h ^ 1], row, un);
                load_v(v[h ^ 1], un);
              } else {
                load(in[0], row, u);
                load_v(v[0], u);
              }
              work(in[DB ? h : 0], v[DB ? h : 0], u, sweep, lop, row, part, sum);
            }
          }
        }
        if (sweep == 0) sum = row_sum(part);
      }
    }
  }
}

// Softmax backward on the rotated format, P = bf16(WHT128(bf16(Y'))) blockwise (the rotated
// decode's result): the two sweeps of k_softmax_2s over the row's rotation blocks instead of
// its units.  Wave w takes items w, w + NW, ... of the row, an item being one 128-column
// rotation block of every plane (128/G units).  Per item and plane a lane rebuilds row j's 32
// columns, gathers them (rot_gather_128) and rotates them in registers (wht128_regs), so P is
// the decode's bit for bit and sits in lane group g at block columns 32g .. 32g+31, where dP is
// read and dS written (four 16-byte pieces per lane and plane).  Sweep 1 sums P dP per row (the
// lane's columns, the row's four lanes, then the waves in order through LDS), sweep 2 rebuilds
// P and writes dS = P (dP - sum).  A wave reads an item's dP before writing its dS, and no other
// wave touches those columns, so dS may overwrite dP.  Planes of whole rotation blocks
// ((N / NP) % 128 == 0).  Rows past the end repeat the last row (identical stores).
//   HOLD > 0 (1 .. HOLD items per wave; one workgroup per CU walking its row blocks): the
//            items' V operands are parked in the wave's LDS slots at the start; the wave keeps
//            its items' codes, qparams and dP of a row block for both sweeps (read once), and
//            requests each item's inputs of the next block as soon as the second sweep has
//            used them.
//   HOLD = 0 (any width): each item's inputs, V operands included, are requested right before
//            the item is computed, in both sweeps.
// (Measured alternatives, MI355X, 16384 x 4096 int4/g64 rank 16: P kept in LDS between the
// sweeps with V read per plane spilled registers, 122 us; without the next-block requests and
// with a workgroup per row block, 115 us; this form 103 us.)
template <int BITS, int G, int R, int NW, int HOLD>
struct SmxRot {
  static constexpr int NP = 8 / BITS, RT = R > 0 ? R / 16 : 1, U = 128 / G;
  static constexpr int VSLOT = U * NP * (G / 16) * RT * 64 * 8;  // one item's V operands in LDS
  static constexpr size_t LDS = (HOLD > 0 && R > 0) ? (size_t)NW * HOLD * VSLOT : 0;
  static_assert(LDS <= 160 * 1024, "LDS budget");
};

template <int BITS, int G, int R, int NW, int HOLD>
__global__ __launch_bounds__(NW * 64) void k_softmax_rot(
    const uint8_t* __restrict__ codes, int64_t ldc, const uint16_t* __restrict__ qparams, int64_t ldq,
    const uint16_t* __restrict__ Lin, int64_t ldl, const uint16_t* __restrict__ V, int M, int N,
    const uint16_t* dp, int64_t lddp, uint16_t* ds, int64_t ldds, int RBW) {
  using Sm = SmxRot<BITS, G, R, NW, HOLD>;
  constexpr int NP = Sm::NP, RT = Sm::RT, E = G / 4, U = Sm::U;
  __shared__ float red[NW][16];
  extern __shared__ __attribute__((aligned(16))) unsigned char vsm[];  // HOLD, R > 0: [NW][HOLD][VSLOT]
  const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int j = lane & 15, g = lane >> 4;
  const int nrb = (M + 15) / 16;
  const int items = N / (NP * 128);
  const int nmine = (items - w + NW - 1) / NW;  // items of this wave (0 when items < NW and w >= items)
  const int PW = N / NP;                        // plane width
  u32x4 wop[2][2];
#pragma unroll
  for (int q0 = 0; q0 < 2; ++q0)
#pragma unroll
    for (int n = 0; n < 2; ++n) wop[q0][n] = wht_base_operand(j, rot_sign_group<G>(g), q0, n != 0);
  struct In {
    u32x4 cb[U][G / 64];
    uint32_t qp[U][NP];
    u32x4 d[NP][4];
  };
  using Vop = u32x2[U][NP][G / 16][RT];
  auto load = [&](In& in, int64_t row, int it) __attribute__((always_inline)) {
#pragma unroll
    for (int ul = 0; ul < U; ++ul) {
      const int u = it * U + ul;
#pragma unroll
      for (int i = 0; i < G / 64; ++i) in.cb[ul][i] = ld16_stream(codes + row * ldc + u * G + E * g + 16 * i);
      if constexpr (NP == 2) {
        const u32x2 q = ld8(qparams + row * ldq + u * 4);
        in.qp[ul][0] = q[0];
        in.qp[ul][1] = q[1];
      } else {
        in.qp[ul][0] = ld4(qparams + row * ldq + u * 2);
      }
    }
#pragma unroll
    for (int p = 0; p < NP; ++p)
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const uint16_t* a = dp + row * lddp + p * PW + it * 128 + 32 * g + 8 * k;
        in.d[p][k] = HOLD > 0 ? ld16_stream(a) : ld16(a);
      }
  };
  auto load_v = [&](Vop& v, int it) __attribute__((always_inline)) {
    if constexpr (R > 0) {
#pragma unroll
      for (int ul = 0; ul < U; ++ul)
#pragma unroll
        for (int p = 0; p < NP; ++p) load_vops<G, R>(V, unit_base(p, it * U + ul, N, NP, G), j, g, v[ul][p]);
    }
  };
  // the LDS slot of held item h of this wave; operand (ul, p, q, t) is 64 lanes x 8 bytes
  auto vslot = [&](int h) { return reinterpret_cast<u32x2*>(vsm + ((size_t)w * HOLD + h) * Sm::VSLOT); };
  constexpr int NOPS = U * NP * (G / 16) * RT;
  auto read_v = [&](Vop& v, int h) __attribute__((always_inline)) {
    if constexpr (R > 0) {
      const u32x2* sl = vslot(h);
      u32x2* f = &v[0][0][0][0];
#pragma unroll
      for (int o = 0; o < NOPS; ++o) f[o] = sl[o * 64 + lane];
    }
  };
  // sweep 0: part += P * dP over the lane's columns; sweep 1: dS = P (dP - sum)
  auto work = [&](const In& in, const Vop& v, int it, int sweep, const u32x2* lop, int64_t row, float& part,
                  float sum) __attribute__((always_inline)) {
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      float xh[32];
#pragma unroll
      for (int ul = 0; ul < U; ++ul) reconstruct_plane<BITS, G, R>(in.cb[ul], in.qp[ul][p], p, v[ul][p], lop, xh + E * ul);
      u32x4 xv[4];
      rot_gather_128<G>(xh, xv);
      float y[32];
      wht128_regs(xv, wop, y);
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        float pr[8], dv[8];
        unpack8(pack8(y + 8 * k), pr);  // P = bf16(rotated), as the decode stores it
        unpack8(in.d[p][k], dv);
        if (sweep == 0) {
#pragma unroll
          for (int e = 0; e < 8; ++e) part = __builtin_fmaf(pr[e], dv[e], part);
        } else {
          float o[8];
#pragma unroll
          for (int e = 0; e < 8; ++e) o[e] = pr[e] * (dv[e] - sum);
          st16(ds + row * ldds + p * PW + it * 128 + 32 * g + 8 * k, pack8(o));
        }
      }
    }
  };
  // the row's four lanes, then the NW waves in order (through LDS)
  auto row_sum = [&](float part) __attribute__((always_inline)) {
    float a = part, c = part;
    swap32(a, c);
    part = a + c;
    a = part, c = part;
    swap16(a, c);
    part = a + c;
    if (g == 0) red[w][j] = part;
    lds_barrier();
    float sum = 0.f;
#pragma unroll
    for (int w2 = 0; w2 < NW; ++w2) sum += red[w2][j];
    lds_barrier();  // every wave has read red before the next row block rewrites it
    return sum;
  };
  const int rb_beg = blockIdx.x * RBW, rb_end = min(nrb, rb_beg + RBW);
  auto load_lop = [&](u32x2* lop, int64_t row) __attribute__((always_inline)) {
    if constexpr (R > 0) {
#pragma unroll
      for (int t = 0; t < RT; ++t) lop[t] = ld8(Lin + row * ldl + 16 * t + 4 * g);
    }
  };
  if constexpr (HOLD > 0) {
    if constexpr (R > 0) {
      // park this wave's V operands (the host launches this form only when 1 <= nmine <= HOLD);
      // a wave reads back only the slots it wrote, in order, so no barrier is needed
#pragma unroll
      for (int h = 0; h < HOLD; ++h) {
        if (h < nmine) {
          Vop v;
          load_v(v, w + h * NW);
          u32x2* sl = vslot(h);
          const u32x2* f = &v[0][0][0][0];
#pragma unroll
          for (int o = 0; o < NOPS; ++o) sl[o * 64 + lane] = f[o];
        }
      }
    }
    In in[HOLD];
    u32x2 lop[RT], lopn[RT];
    if (rb_beg < rb_end) {
      const int64_t row0 = min(rb_beg * 16 + j, M - 1);
      load_lop(lop, row0);
#pragma unroll
      for (int h = 0; h < HOLD; ++h) load(in[h], row0, w + min(h, nmine - 1) * NW);
    }
#pragma unroll 1
    for (int rb = rb_beg; rb < rb_end; ++rb) {
      const int64_t row = min(rb * 16 + j, M - 1);
      const bool more = rb + 1 < rb_end;  // wave-uniform
      const int64_t rown = min((rb + 1) * 16 + j, M - 1);
      float part = 0.f;
#pragma unroll
      for (int h = 0; h < HOLD; ++h) {
        if (h < nmine) {  // wave-uniform
          Vop v;
          read_v(v, h);
          work(in[h], v, w + h * NW, 0, lop, row, part, 0.f);
        }
      }
      const float sum = row_sum(part);
      if (more) load_lop(lopn, rown);
#pragma unroll
      for (int h = 0; h < HOLD; ++h) {
        if (h < nmine) {
          Vop v;
          read_v(v, h);
          work(in[h], v, w + h * NW, 1, lop, row, part, sum);
        }
        // this item's inputs of the next block, while the rest of this block is computed
        if (more) load(in[h], rown, w + min(h, nmine - 1) * NW);
      }
#pragma unroll
      for (int t = 0; t < RT; ++t) lop[t] = lopn[t];
    }
  } else {
#pragma unroll 1
    for (int rb = rb_beg; rb < rb_end; ++rb) {
      const int64_t row = min(rb * 16 + j, M - 1);
      u32x2 lop[RT];
      load_lop(lop, row);
      float part = 0.f, sum = 0.f;
#pragma unroll 1
      for (int sweep = 0; sweep < 2; ++sweep) {
#pragma unroll 1
        for (int it = w; it < items; it += NW) {  // wave-uniform
          In in;
          Vop v;
          load(in, row, it);
          load_v(v, it);
          work(in, v, it, sweep, lop, row, part, sum);
        }
        if (sweep == 0) sum = row_sum(part);
      }
    }
  }
}

// Row-persistent softmax backward (one workgroup per CU; wave w owns unit w of every row, so
// a workgroup holds whole rows).  dP moves as whole row segments straight from HBM into an LDS
// tile (two tiles, block b in tile b&1), is read back in the MFMA layout, and dS is written
// over it in the same layout; after the next barrier the workgroup stores the tile as whole
// row segments (non-temporal, full lines).  Codes, qparams and L of the wave's unit come one
// block ahead in registers.  Per block: barrier (block b's dP visible, block b-1's dS
// complete) -> store block b-1's tile -> barrier (its reads returned) -> dP of block b+1 into
// that tile -> reconstruct, row sums (one more barrier), dS.  Rows past the end repeat the
// last row (identical stores).
template <int BITS, int G, int NW>
struct SmxTile {
  static constexpr int NP = 8 / BITS;
  static constexpr int ROWB = NW * G * NP * 2;  // bytes of a bf16 row (the workgroup's NW units)
  static constexpr int PITCH = ROWB + 16;       // LDS row pitch (spreads the 16 rows over banks)
  static constexpr int TILE = 16 * PITCH;
  static constexpr int CPR = ROWB / 1024;       // 1 KB chunks per row
  static constexpr int DPW = 16 * CPR / NW;     // dP loads per wave and block
  static constexpr int SPT = 16 * ROWB / 16 / (NW * 64);  // 16-byte tile chunks per thread
  static constexpr size_t LDS = 2 * (size_t)TILE + (size_t)NW * 16 * 4;
  static_assert(ROWB % 1024 == 0 && (16 * CPR) % NW == 0 && (16 * ROWB / 16) % (NW * 64) == 0, "tile split");
  static_assert(LDS <= 160 * 1024, "LDS budget");
};

template <int BITS, int G, int R, int NW>
__global__ __launch_bounds__(NW * 64) void k_softmax_rows(
    const uint8_t* __restrict__ codes, int64_t ldc, const uint16_t* __restrict__ qparams, int64_t ldq,
    const uint16_t* __restrict__ Lin, int64_t ldl, const uint16_t* __restrict__ V, int M, int N,
    const uint16_t* __restrict__ dp, int64_t lddp, uint16_t* __restrict__ ds, int64_t ldds, int RBW) {
  using St = SmxTile<BITS, G, NW>;
  constexpr int NP = St::NP, RT = R > 0 ? R / 16 : 1, E = G / 4;
  extern __shared__ __attribute__((aligned(16))) unsigned char sm[];  // [2][TILE], red
  float* red = reinterpret_cast<float*>(sm + 2 * St::TILE);          // [NW][16]
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int j = lane & 15, g = lane >> 4;
  const int nrb = (M + 15) / 16;
  const int rb0 = blockIdx.x * RBW;
  if (rb0 >= nrb) return;  // whole workgroup
  const int nblk = min(RBW, nrb - rb0);
  const int u = w;

  u32x2 vop[NP][G / 16][RT];
  if constexpr (R > 0) {
#pragma unroll
    for (int p = 0; p < NP; ++p) load_vops<G, R>(V, unit_base(p, u, N, NP, G), j, g, vop[p]);
  }
  struct Cin {
    u32x4 cb[G / 64];
    uint32_t qp[NP];
    u32x2 lop[RT];
  };
  constexpr int kC = G / 64 + 1 + (R > 0 ? RT : 0);  // loads of one cload
  auto cload = [&](Cin& c, int rb) {
    const int64_t row = min(rb * 16 + j, M - 1);
#pragma unroll
    for (int i = 0; i < G / 64; ++i) c.cb[i] = ld16_stream(codes + row * ldc + u * G + E * g + 16 * i);
    if constexpr (NP == 2) {
      const u32x2 q = ld8(qparams + row * ldq + u * 4);
      c.qp[0] = q[0];
      c.qp[1] = q[1];
    } else {
      c.qp[0] = ld4(qparams + row * ldq + u * 2);
    }
    if constexpr (R > 0) {
#pragma unroll
      for (int t = 0; t < RT; ++t) c.lop[t] = ld8(Lin + row * ldl + 16 * t + 4 * g);
    }
  };
  const unsigned char* dpb = reinterpret_cast<const unsigned char*>(dp);
  unsigned char* dsb = reinterpret_cast<unsigned char*>(ds);
  auto dma = [&](int rb, int tb) {
    unsigned char* tile = sm + tb * St::TILE;
#pragma unroll
    for (int i = 0; i < St::DPW; ++i) {
      const int q = w * St::DPW + i, r = q / St::CPR, c = q % St::CPR;
      const int64_t row = min(rb * 16 + r, M - 1);
      ld16_to_lds(dpb + row * lddp * 2 + c * 1024 + lane * 16, tile + r * St::PITCH + c * 1024);
    }
  };
  auto store_tile = [&](int rb, int tb) {
    const unsigned char* tile = sm + tb * St::TILE;
#pragma unroll
    for (int i = 0; i < St::SPT; ++i) {
      const int k = tid + NW * 64 * i, r = k / (St::ROWB / 16), c16 = k % (St::ROWB / 16);
      const u32x4 v = *reinterpret_cast<const u32x4*>(tile + r * St::PITCH + c16 * 16);
      const int64_t row = min(rb * 16 + r, M - 1);
      st16_stream(dsb + row * ldds * 2 + c16 * 16, v);
    }
  };
  // the lane's bf16 columns of plane p, k-th 8-column piece, in the tile
  auto tpos = [&](unsigned char* tile, int p, int k) {
    return reinterpret_cast<u32x4*>(tile + j * St::PITCH + (unit_base(p, u, N, NP, G) + E * g + 8 * k) * 2);
  };
  auto compute = [&](const Cin& c, int tb) {
    unsigned char* tile = sm + tb * St::TILE;
    u32x4 pb[NP][G / 32];  // P = bf16(decode), packed (exact)
    float part = 0.f;
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      float pv[E];
      reconstruct_plane<BITS, G, R>(c.cb, c.qp[p], p, vop[p], c.lop, pv);
#pragma unroll
      for (int k = 0; k < G / 32; ++k) {
        pb[p][k] = pack8(pv + 8 * k);
        float pr[8], dv[8];
        unpack8(pb[p][k], pr);
        unpack8(*tpos(tile, p, k), dv);
#pragma unroll
        for (int e = 0; e < 8; ++e) part = __builtin_fmaf(pr[e], dv[e], part);
      }
    }
    {
      float a = part, b = part;
      swap32(a, b);
      part = a + b;
      a = part, b = part;
      swap16(a, b);
      part = a + b;
    }
    if (g == 0) red[w * 16 + j] = part;
    lds_barrier();
    float sum = 0.f;
#pragma unroll
    for (int w2 = 0; w2 < NW; ++w2) sum += red[w2 * 16 + j];
#pragma unroll
    for (int p = 0; p < NP; ++p)
#pragma unroll
      for (int k = 0; k < G / 32; ++k) {
        float pr[8], dv[8], o[8];
        unpack8(pb[p][k], pr);
        unpack8(*tpos(tile, p, k), dv);
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = pr[e] * (dv[e] - sum);
        *tpos(tile, p, k) = pack8(o);
      }
  };
  auto step = [&](Cin& cur, Cin& nxt, int b) {
    const int tb = b & 1;
    // block b's dP loads are done: after them this wave issued only block b's cload (kC loads);
    // vmcnt retires in issue order on gfx9
    __builtin_amdgcn_s_waitcnt(0x0f70 | kC);
    lds_barrier();
    if (b > 0) store_tile(rb0 + b - 1, tb ^ 1);
    if (b + 1 < nblk) {
      lds_barrier();  // every wave's reads of tile tb^1 have returned
      __builtin_amdgcn_sched_barrier(0);
      dma(rb0 + b + 1, tb ^ 1);
      __builtin_amdgcn_sched_barrier(0);
      cload(nxt, rb0 + b + 1);
      __builtin_amdgcn_sched_barrier(0);
    }
    compute(cur, tb);
  };
  static_assert(kC < 16, "vmcnt immediate");
  Cin cin[2];
  dma(rb0, 0);
  __builtin_amdgcn_sched_barrier(0);
  cload(cin[0], rb0);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll 1
  for (int b = 0; b < nblk; b += 2) {
    step(cin[0], cin[1], b);
    if (b + 1 < nblk) step(cin[1], cin[0], b + 1);
  }
  lds_barrier();
  store_tile(rb0 + nblk - 1, (nblk - 1) & 1);
}

// ------------------------------------------------------------------ dequant-GEMM
// Grid: ceil(row blocks / RBW); NW waves; wave w takes units w, w + NW, ...; for each unit
// it decodes the RBW row blocks and multiplies them into its partial out tiles (A's MFMA
// operand is regenerated per unit with the identity-MFMA transpose of lrq_common.h).  A unit's
// inputs sit in one of SL register slots, loaded while the previous unit is computed.  The NW
// partial tiles of a row block are then summed through LDS, each wave summing 1/NW of it.
// Outlier channels in the dequant-GEMMs: x_hat[:, idx] = bf16(side), so
//   out = sum over the other columns of x_hat A  +  bf16(side) @ A[idx, :].
// The first sum is the ordinary kernel with A's operand rows of outlier columns zeroed (once);
// the second enters the same fp32 accumulators as extra K entries (one 16x16x32 step per 32
// side columns, added by wave 0 per row block): the products and the accumulation are those
// of the decoded activation's GEMM.  Up to kSideGemmMax side columns.
constexpr int kSideGemmMax = 64;

template <int TO>
struct SideGemm {
  static constexpr int KC = kSideGemmMax / 32;
  // lane (i, g), chunk m, tile t: A[idx[32m + 8g + e]][16t + i], e < 8 (0 past nout and for an
  // index outside [0, N), which the decode ignores too)
  u32x4 a[KC][TO];
  __device__ __forceinline__ void load_a(const uint16_t* __restrict__ A, int n_out, int N,
                                         const int32_t* __restrict__ oidx, int nout, int i, int g) {
#pragma unroll
    for (int m = 0; m < KC; ++m)
#pragma unroll
      for (int t = 0; t < TO; ++t) {
        uint32_t h[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int sc = 32 * m + 8 * g + e;
          const int c = oidx[min(sc, nout - 1)];
          const bool ok = sc < nout && c >= 0 && c < N;
          const uint16_t v = A[(int64_t)(ok ? c : 0) * n_out + 16 * t + i];
          h[e] = ok ? v : 0u;
        }
        a[m][t] = u32x4{h[0] | (h[1] << 16), h[2] | (h[3] << 16), h[4] | (h[5] << 16), h[6] | (h[7] << 16)};
      }
  }
  // the lane's side values of row `row` for every chunk (columns past nout clamp to a valid one)
  __device__ static __forceinline__ void load_b(uint32_t (&sd)[KC][8], const uint16_t* __restrict__ side,
                                                int64_t ldside, int64_t row, int nout, int g) {
#pragma unroll
    for (int m = 0; m < KC; ++m)
#pragma unroll
      for (int e = 0; e < 8; ++e) sd[m][e] = side[row * ldside + min(32 * m + 8 * g + e, nout - 1)];
  }
  __device__ __forceinline__ void apply(const uint32_t (&sd)[KC][8], f32x4* acc, int nout) const {
#pragma unroll
    for (int m = 0; m < KC; ++m) {
      if (32 * m >= nout) break;  // uniform
      float f[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) f[e] = f16_val(sd[m][e]);
      const u32x4 b = pack8(f);  // bf16(side), as the decode returns it
#pragma unroll
      for (int t = 0; t < TO; ++t) acc[t] = mfma_16x16x32(a[m][t], b, acc[t]);
    }
  }
};

// acc[b * TO + t] += side term of row block rb0 + b, tile t (after the main loop, so the side
// operands hold no registers while the units are walked).
template <int TO, int RBW>
__device__ __forceinline__ void add_side_term(const uint16_t* __restrict__ A, int n_out, int N,
                                              const int32_t* __restrict__ oidx, int nout,
                                              const uint16_t* __restrict__ side, int64_t ldside, int rb0, int nrb,
                                              int M, int j, int g, f32x4* acc) {
  SideGemm<TO> sg;
  sg.load_a(A, n_out, N, oidx, nout, j, g);
#pragma unroll
  for (int b = 0; b < RBW; ++b) {
    uint32_t sd[SideGemm<TO>::KC][8];
    SideGemm<TO>::load_b(sd, side, ldside, min(min(rb0 + b, nrb - 1) * 16 + j, M - 1), nout, g);
    sg.apply(sd, acc + b * TO, nout);
  }
}

// Column mask of the outlier channels in LDS (N/32 words), built by the whole workgroup.
__device__ __forceinline__ void build_colmask(uint32_t* mask, int N, const int32_t* __restrict__ oidx, int nout) {
  for (int i = threadIdx.x; i < N / 32; i += blockDim.x) mask[i] = 0u;
  __syncthreads();
  for (int k = threadIdx.x; k < nout; k += blockDim.x) {
    const int c = oidx[k];
    if (c >= 0 && c < N) atomicOr(&mask[c >> 5], 1u << (c & 31));
  }
  __syncthreads();
}

// Zero the operand rows (lane (j, g) of operand q holds row vrow_res(base, j, q)) of outlier columns.
template <int G, int T>
__device__ __forceinline__ void mask_rows(u32x2 (&op)[G / 16][T], const uint32_t* mask, int base, int j) {
#pragma unroll
  for (int q = 0; q < G / 16; ++q) {
    const int c = vrow_res<G>(base, j, q);
    const bool z = (mask[c >> 5] >> (c & 31)) & 1u;
#pragma unroll
    for (int t = 0; t < T; ++t) op[q][t] = z ? u32x2{0u, 0u} : op[q][t];
  }
}

template <int BITS, int G, int R, int NOUT, int NW, int RBW, int SL, bool OUT_F32, bool OUTL>
__global__ __launch_bounds__(NW * 64) void k_dequant_gemm(
    const uint8_t* __restrict__ codes, int64_t ldc, const uint16_t* __restrict__ qparams, int64_t ldq,
    const uint16_t* __restrict__ Lin, int64_t ldl, const uint16_t* __restrict__ V, int M, int N,
    const uint16_t* __restrict__ A, void* __restrict__ out, int64_t ldo, const int32_t* __restrict__ oidx, int nout,
    const uint16_t* __restrict__ side, int64_t ldside) {
  constexpr int NP = 8 / BITS, RT = R > 0 ? R / 16 : 1, TO = NOUT / 16, E = G / 4;
  __shared__ f32x4 part[NW][TO][64];
  extern __shared__ uint32_t gmask[];  // OUTL: N/32 words
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int j = lane & 15, g = lane >> 4;
  const int nrb = (M + 15) / 16;
  const int rb0 = blockIdx.x * RBW;
  const int units = N / (G * NP);
  const u32x2 ident = identity_bop(j, g);
  if constexpr (OUTL) build_colmask(gmask, N, oidx, nout);

  f32x4 acc[RBW][TO];
#pragma unroll
  for (int b = 0; b < RBW; ++b)
#pragma unroll
    for (int t = 0; t < TO; ++t) acc[b][t] = zero4();

  // L of the RBW row blocks (the same for every unit)
  u32x2 lop[RBW][RT];
#pragma unroll
  for (int b = 0; b < RBW; ++b) {
    const int64_t row = min(min(rb0 + b, nrb - 1) * 16 + j, M - 1);
    if constexpr (R > 0) {
#pragma unroll
      for (int t = 0; t < RT; ++t) lop[b][t] = ld8(Lin + row * ldl + 16 * t + 4 * g);
    }
  }
  // per unit: V and A operands, codes and qparams of the RBW blocks; the wave's units
  // w, w + NW, ... go through SL register slots, the next unit's loads in flight while one
  // is computed (clamped unit index for the slots past the wave's last unit)
  struct UIn {
    u32x2 vop[NP][G / 16][RT];
    u32x2 va[NP][G / 16][TO];
    u32x4 cb[RBW][G / 64];
    uint32_t qp[RBW][NP];
  };
  auto load_unit = [&](int u, UIn& d) {
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      if constexpr (R > 0) load_vops<G, R>(V, unit_base(p, u, N, NP, G), j, g, d.vop[p]);
      load_vops<G, NOUT>(A, unit_base(p, u, N, NP, G), j, g, d.va[p]);
      if constexpr (OUTL) mask_rows<G, TO>(d.va[p], gmask, unit_base(p, u, N, NP, G), j);
    }
#pragma unroll
    for (int b = 0; b < RBW; ++b) {
      const int64_t row = min(min(rb0 + b, nrb - 1) * 16 + j, M - 1);
#pragma unroll
      for (int i = 0; i < G / 64; ++i) d.cb[b][i] = ld16_stream(codes + row * ldc + u * G + E * g + 16 * i);
      if constexpr (NP == 2) {
        const u32x2 q = ld8(qparams + row * ldq + u * 4);
        d.qp[b][0] = q[0];
        d.qp[b][1] = q[1];
      } else {
        d.qp[b][0] = ld4(qparams + row * ldq + u * 2);
      }
    }
  };
  auto compute_unit = [&](const UIn& d) {
#pragma unroll
    for (int b = 0; b < RBW; ++b)
#pragma unroll
      for (int p = 0; p < NP; ++p) {
        float xh[E];
        reconstruct_plane<BITS, G, R>(d.cb[b], d.qp[b][p], p, d.vop[p], lop[b], xh);
        u32x4 xb[G / 32];
#pragma unroll
        for (int k = 0; k < G / 32; ++k) xb[k] = pack8(xh + 8 * k);  // x_hat = bf16(reconstruction)
        project_unit<G, NOUT>(d.va[p], xb, ident, acc[b]);
      }
  };
  const int nu = w < units ? (units - w + NW - 1) / NW : 0;
  UIn ring[SL];
#pragma unroll
  for (int sl = 0; sl < SL; ++sl) load_unit(min(w + sl * NW, units - 1), ring[sl]);
  for (int i0 = 0; i0 < nu; i0 += SL) {
#pragma unroll
    for (int sl = 0; sl < SL; ++sl) {
      if (i0 + sl < nu) compute_unit(ring[sl]);  // wave-uniform; no memory operation inside
      load_unit(min(w + (i0 + sl + SL) * NW, units - 1), ring[sl]);
    }
  }
  if constexpr (OUTL) {
    if (w == 0) add_side_term<TO, RBW>(A, NOUT, N, oidx, nout, side, ldside, rb0, nrb, M, j, g, &acc[0][0]);
  }

  // acc[b][t] in lane (j, g), component v: out[row j][16t + 4g + v] (partial over this wave's units)
  constexpr int F = TO * 256 / NW, S = 64 / F, PPL = NW / S;
  static_assert(F >= 1 && F <= 64 && 64 % F == 0 && NW % S == 0, "out reduction split");
  const float* partf = reinterpret_cast<const float*>(&part[0][0][0]);
#pragma unroll
  for (int b = 0; b < RBW; ++b) {
    if (rb0 + b >= nrb) break;  // uniform
#pragma unroll
    for (int t = 0; t < TO; ++t) part[w][t][lane] = acc[b][t];
    __syncthreads();
    const int f = lane % F, pg = lane / F;
    const int fi = w * F + f;
    const int t = fi >> 8, src = (fi >> 2) & 63, v = fi & 3;
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < PPL; ++i) s += partf[(((pg * PPL + i) * TO + t) * 64 + src) * 4 + v];
#pragma unroll
    for (int m = F; m < 64; m <<= 1) s += __shfl_xor(s, m);
    const int row = (rb0 + b) * 16 + (src & 15);
    const int col = 16 * t + 4 * (src >> 4) + v;
    if (pg == 0 && row < M) {
      if constexpr (OUT_F32) reinterpret_cast<float*>(out)[(int64_t)row * ldo + col] = s;
      else reinterpret_cast<uint16_t*>(out)[(int64_t)row * ldo + col] = (uint16_t)pack_bf16x2(s, 0.f);
    }
    __syncthreads();
  }
}

// Dequant-GEMM on the rotated format with the rotation in registers (no LDS tile, no barrier
// until the final reduction).  Wave w takes the pairs (item, plane) w, w + NW, ... of the row,
// an item being one 128-column rotation block (128/G units); per pair it walks the workgroup's
// RBW row blocks, rebuilding row j's 32 columns of the block, gathering them (rot_gather_128)
// and rotating them (wht128_regs), so x_hat is the decode's bit for bit and lane group g holds
// block columns 32g .. 32g+31 as four 8-column chunks.  Chunk c is the B operand of a 16x16x32
// step whose A operand holds A[column 32g + 8c + e][16t + i] in lane (i, g) (gathered once per
// pair; zero for outlier columns, whose side term is added at the end as in k_dequant_gemm),
// so the accumulator holds out[row j][16t + 4g + v] as in k_dequant_gemm.  The next row block's
// codes and qparams are requested before the current one is computed.  The waves' partial tiles
// are summed through LDS in wave order.  Planes of whole rotation blocks ((N / NP) % 128 == 0).
template <int BITS, int G, int R, int NOUT, int NW, int RBW, bool OUT_F32, bool OUTL>
__global__ __launch_bounds__(NW * 64) void k_dequant_gemm_rotr(
    const uint8_t* __restrict__ codes, int64_t ldc, const uint16_t* __restrict__ qparams, int64_t ldq,
    const uint16_t* __restrict__ Lin, int64_t ldl, const uint16_t* __restrict__ V, int M, int N,
    const uint16_t* __restrict__ A, void* __restrict__ out, int64_t ldo, const int32_t* __restrict__ oidx, int nout,
    const uint16_t* __restrict__ side, int64_t ldside) {
  constexpr int NP = 8 / BITS, RT = R > 0 ? R / 16 : 1, TO = NOUT / 16, E = G / 4, U = 128 / G;
  __shared__ f32x4 part[NW][TO][64];
  extern __shared__ uint32_t gmask[];  // OUTL: N/32 words
  const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int j = lane & 15, g = lane >> 4;
  const int nrb = (M + 15) / 16;
  const int rb0 = blockIdx.x * RBW;
  const int PW = N / NP;
  const int pairs = (N / (NP * 128)) * NP;
  if constexpr (OUTL) build_colmask(gmask, N, oidx, nout);
  u32x4 wop[2][2];
#pragma unroll
  for (int q0 = 0; q0 < 2; ++q0)
#pragma unroll
    for (int n = 0; n < 2; ++n) wop[q0][n] = wht_base_operand(j, rot_sign_group<G>(g), q0, n != 0);

  f32x4 acc[RBW][TO];
#pragma unroll
  for (int b = 0; b < RBW; ++b)
#pragma unroll
    for (int t = 0; t < TO; ++t) acc[b][t] = zero4();
  u32x2 lop[RBW][RT];
#pragma unroll
  for (int b = 0; b < RBW; ++b) {
    const int64_t row = min(min(rb0 + b, nrb - 1) * 16 + j, M - 1);
    if constexpr (R > 0) {
#pragma unroll
      for (int t = 0; t < RT; ++t) lop[b][t] = ld8(Lin + row * ldl + 16 * t + 4 * g);
    }
  }
  struct Blk {
    u32x4 cb[U][G / 64];
    uint32_t qp[U];
  };
  // (item it, plane p) of row block b: the U units' code bytes of row j and plane p's (scale, zero)
  auto load = [&](int it, int p, int b, Blk& d) __attribute__((always_inline)) {
    const int64_t row = min(min(rb0 + b, nrb - 1) * 16 + j, M - 1);
#pragma unroll
    for (int ul = 0; ul < U; ++ul) {
      const int u = it * U + ul;
#pragma unroll
      for (int i = 0; i < G / 64; ++i) d.cb[ul][i] = ld16_stream(codes + row * ldc + u * G + E * g + 16 * i);
      d.qp[ul] = ld4(qparams + row * ldq + (u * NP + p) * 2);
    }
  };
  // the pair's operands: V of the U units (reconstruction) and the gathered A chunks
  struct Ops {
    u32x2 vop[U][G / 16][RT];
    u32x4 ach[4][TO];
  };
  auto load_ops = [&](int pi, Ops& o) __attribute__((always_inline)) {
    const int it = pi / NP, p = pi % NP;
    if constexpr (R > 0) {
#pragma unroll
      for (int ul = 0; ul < U; ++ul) load_vops<G, R>(V, unit_base(p, it * U + ul, N, NP, G), j, g, o.vop[ul]);
    }
    const int c0 = p * PW + it * 128 + 32 * g;
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
      for (int t = 0; t < TO; ++t) {
        uint32_t h[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int col = c0 + 8 * c + e;
          uint32_t v = A[(int64_t)col * NOUT + 16 * t + j];
          if constexpr (OUTL) v = ((gmask[col >> 5] >> (col & 31)) & 1u) ? 0u : v;
          h[e] = v;
        }
        o.ach[c][t] = u32x4{h[0] | (h[1] << 16), h[2] | (h[3] << 16), h[4] | (h[5] << 16), h[6] | (h[7] << 16)};
      }
  };
  static_assert(RBW % 2 == 0, "block b of every pair in ring slot b % 2");
  // PF: the next pair's operands and first block are requested during the current pair's last
  // block (a second operand set; at rank 32 it would not fit beside the rest)
  constexpr bool PF = R <= 16;
  const int np_mine = w < pairs ? (pairs - w + NW - 1) / NW : 0;
  Ops ops[PF ? 2 : 1];
  Blk ring[2];
  auto pair = [&](auto par_tag, int k) __attribute__((always_inline)) {
    constexpr int par = decltype(par_tag)::value;
    Ops& o = ops[PF ? par : 0];
    const int pi = w + k * NW, it = pi / NP, p = pi % NP;
    const bool more = k + 1 < np_mine;  // wave-uniform
    if constexpr (!PF) {
      load_ops(pi, o);
      load(it, p, 0, ring[0]);
    }
    static_for<0, RBW>([&](auto bc) {
      constexpr int b = decltype(bc)::value;
      if constexpr (b + 1 < RBW) {
        load(it, p, b + 1, ring[(b + 1) & 1]);
      } else if constexpr (PF) {
        if (more) {
          const int pn = pi + NW;
          load_ops(pn, ops[par ^ 1]);
          load(pn / NP, pn % NP, 0, ring[0]);
        }
      }
      const Blk& cur = ring[b & 1];
      float xh[32];
#pragma unroll
      for (int ul = 0; ul < U; ++ul) reconstruct_plane<BITS, G, R>(cur.cb[ul], cur.qp[ul], p, o.vop[ul], lop[b], xh + E * ul);
      u32x4 xv[4];
      rot_gather_128<G>(xh, xv);
      float y[32];
      wht128_regs(xv, wop, y);
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const u32x4 xc = pack8(y + 8 * c);  // x_hat of row j, block columns 32g + 8c .. +7
#pragma unroll
        for (int t = 0; t < TO; ++t) acc[b][t] = mfma_16x16x32(o.ach[c][t], xc, acc[b][t]);
      }
    });
  };
  if (PF && np_mine > 0) {
    load_ops(w, ops[0]);
    load(w / NP, w % NP, 0, ring[0]);
  }
#pragma unroll 1
  for (int k = 0; k < np_mine; k += 2) {
    pair(std::integral_constant<int, 0>{}, k);
    if (k + 1 < np_mine) pair(std::integral_constant<int, 1>{}, k + 1);
  }
  if constexpr (OUTL) {
    if (w == 0) add_side_term<TO, RBW>(A, NOUT, N, oidx, nout, side, ldside, rb0, nrb, M, j, g, &acc[0][0]);
  }

  // acc[b][t] in lane (j, g), component v: out[row j][16t + 4g + v] (as in k_dequant_gemm)
  constexpr int F = TO * 256 / NW, S = 64 / F, PPL = NW / S;
  static_assert(F >= 1 && F <= 64 && 64 % F == 0 && NW % S == 0, "out reduction split");
  const float* partf = reinterpret_cast<const float*>(&part[0][0][0]);
#pragma unroll
  for (int b = 0; b < RBW; ++b) {
    if (rb0 + b >= nrb) break;  // uniform
#pragma unroll
    for (int t = 0; t < TO; ++t) part[w][t][lane] = acc[b][t];
    __syncthreads();
    const int f = lane % F, pg = lane / F;
    const int fi = w * F + f;
    const int t = fi >> 8, src = (fi >> 2) & 63, v = fi & 3;
    float sum = 0.f;
#pragma unroll
    for (int i = 0; i < PPL; ++i) sum += partf[(((pg * PPL + i) * TO + t) * 64 + src) * 4 + v];
#pragma unroll
    for (int m = F; m < 64; m <<= 1) sum += __shfl_xor(sum, m);
    const int row = (rb0 + b) * 16 + (src & 15);
    const int col = 16 * t + 4 * (src >> 4) + v;
    if (pg == 0 && row < M) {
      if constexpr (OUT_F32) reinterpret_cast<float*>(out)[(int64_t)row * ldo + col] = sum;
      else reinterpret_cast<uint16_t*>(out)[(int64_t)row * ldo + col] = (uint16_t)pack_bf16x2(sum, 0.f);
    }
    __syncthreads();
  }
}

// Dequant-GEMM for n = 16 when the row's units split evenly over the waves (NU per wave):
// wave w owns units NU*w .. NU*w + NU-1 and keeps their reconstruction operands and the
// transposed A operands in registers for the whole kernel (loaded and transposed once, not per
// unit visit as in k_dequant_gemm).  It walks the workgroup's RBW row blocks with the codes,
// qparams and L of the next SL blocks in flight; the block loop is unrolled, so every slot and
// accumulator index is static and blocks past the last one issue no loads.  Rows past the end
// repeat the last row (their sums are not stored).  The 8 partial tiles of a block are summed
// through LDS in wave order as in k_dequant_gemm.
template <int BITS, int G, int R, int NW, int NU, int RBW, int SL, bool OUT_F32, bool OUTL>
__global__ __launch_bounds__(NW * 64) void k_dequant_gemm_w(
    const uint8_t* __restrict__ codes, int64_t ldc, const uint16_t* __restrict__ qparams, int64_t ldq,
    const uint16_t* __restrict__ Lin, int64_t ldl, const uint16_t* __restrict__ V, int M, int N,
    const uint16_t* __restrict__ A, void* __restrict__ out, int64_t ldo, const int32_t* __restrict__ oidx, int nout,
    const uint16_t* __restrict__ side, int64_t ldside) {
  constexpr int NP = 8 / BITS, RT = R > 0 ? R / 16 : 1, E = G / 4;
  static_assert(R == 0 || R == 16, "rank 0 or 16");
  __shared__ f32x4 part[NW][64];
  extern __shared__ uint32_t gmask[];  // OUTL: N/32 words
  const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int j = lane & 15, g = lane >> 4;
  const int nrb = (M + 15) / 16;
  const int rb0 = blockIdx.x * RBW;
  const int ub = w * NU;
  const u32x2 ident = identity_bop(j, g);
  if constexpr (OUTL) build_colmask(gmask, N, oidx, nout);

  u32x2 vop[NU][NP][G / 16][RT];
  u32x4 vt[NU][NP][G / 32][1];

  struct BIn {
    u32x4 cb[NU][G / 64];
    uint32_t qp[NU][NP];
    u32x2 lop[RT];
  };
  auto load_blk = [&](int rb, BIn& d) {
    const int64_t row = min(min(rb, nrb - 1) * 16 + j, M - 1);
#pragma unroll
    for (int uu = 0; uu < NU; ++uu) {
#pragma unroll
      for (int i = 0; i < G / 64; ++i) d.cb[uu][i] = ld16_stream(codes + row * ldc + (ub + uu) * G + E * g + 16 * i);
      if constexpr (NP == 2) {
        const u32x2 q = ld8(qparams + row * ldq + (ub + uu) * 4);
        d.qp[uu][0] = q[0];
        d.qp[uu][1] = q[1];
      } else {
        d.qp[uu][0] = ld4(qparams + row * ldq + (ub + uu) * 2);
      }
    }
    if constexpr (R > 0) {
#pragma unroll
      for (int t = 0; t < RT; ++t) d.lop[t] = ld8(Lin + row * ldl + 16 * t + 4 * g);
    }
  };
  auto compute_blk = [&](const BIn& d, f32x4& acc) {
#pragma unroll
    for (int uu = 0; uu < NU; ++uu)
#pragma unroll
      for (int p = 0; p < NP; ++p) {
        float xh[E];
        reconstruct_plane<BITS, G, R>(d.cb[uu], d.qp[uu][p], p, vop[uu][p], d.lop, xh);
        u32x4 xb[G / 32];
#pragma unroll
        for (int k = 0; k < G / 32; ++k) xb[k] = pack8(xh + 8 * k);  // x_hat = bf16(reconstruction)
        project_unit_vt<G, 16>(vt[uu][p], xb, &acc);
      }
  };

  // The first SL blocks' loads go out before the operand set-up, so their latency overlaps it.
  // Where the resident operands and the slots fit the register budget together, the operand
  // loads all go out before the first transpose (one round trip) and the resident operands are
  // pinned: otherwise the compiler may reload them per block, and the wait for such a reload
  // would also drain every block load issued before it.  Else each unit-plane is loaded and
  // transposed in turn, and the compiler's reloads are the cheaper choice.
  constexpr int kResident = NU * NP * ((R > 0 ? G / 16 * RT * 2 : 0) + G / 32 * 4);
  constexpr int kSlots = SL * (NU * (G / 64) * 4 + NU * NP + 2 * RT);
  constexpr bool kPin = kResident + kSlots <= 190;
  f32x4 acc[RBW];
  BIn ring[SL];
#pragma unroll
  for (int sl = 0; sl < SL && sl < RBW; ++sl) load_blk(rb0 + sl, ring[sl]);
  if constexpr (kPin) __builtin_amdgcn_sched_barrier(0);
  if constexpr (kPin) {
    {
      u32x2 va[NU][NP][G / 16][1];
#pragma unroll
      for (int uu = 0; uu < NU; ++uu)
#pragma unroll
        for (int p = 0; p < NP; ++p) {
          const int base = unit_base(p, ub + uu, N, NP, G);
          if constexpr (R > 0) load_vops<G, R>(V, base, j, g, vop[uu][p]);
          load_vops<G, 16>(A, base, j, g, va[uu][p]);
        }
#pragma unroll
      for (int uu = 0; uu < NU; ++uu)
#pragma unroll
        for (int p = 0; p < NP; ++p) {
          if constexpr (OUTL) mask_rows<G, 1>(va[uu][p], gmask, unit_base(p, ub + uu, N, NP, G), j);
          transpose_vops<G, 16>(va[uu][p], ident, vt[uu][p]);
        }
    }
#pragma unroll
    for (int uu = 0; uu < NU; ++uu)
#pragma unroll
      for (int p = 0; p < NP; ++p) {
#pragma unroll
        for (int k = 0; k < G / 32; ++k) pin(vt[uu][p][k][0]);
        if constexpr (R > 0) {
#pragma unroll
          for (int q = 0; q < G / 16; ++q)
#pragma unroll
            for (int t = 0; t < RT; ++t) pin(vop[uu][p][q][t]);
        }
      }
  } else {
#pragma unroll
    for (int uu = 0; uu < NU; ++uu)
#pragma unroll
      for (int p = 0; p < NP; ++p) {
        const int base = unit_base(p, ub + uu, N, NP, G);
        if constexpr (R > 0) load_vops<G, R>(V, base, j, g, vop[uu][p]);
        u32x2 va[G / 16][1];
        load_vops<G, 16>(A, base, j, g, va);
        if constexpr (OUTL) mask_rows<G, 1>(va, gmask, base, j);
        transpose_vops<G, 16>(va, ident, vt[uu][p]);
      }
  }
#pragma unroll
  for (int b = 0; b < RBW; ++b) acc[b] = zero4();
  if constexpr (kPin) __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int b = 0; b < RBW; ++b) {
    compute_blk(ring[b % SL], acc[b]);
    if constexpr (kPin) __builtin_amdgcn_sched_barrier(0);
    if (b + SL < RBW) load_blk(rb0 + b + SL, ring[b % SL]);
    if constexpr (kPin) __builtin_amdgcn_sched_barrier(0);
  }
  if constexpr (OUTL) {
    if (w == 0) add_side_term<1, RBW>(A, 16, N, oidx, nout, side, ldside, rb0, nrb, M, j, g, acc);
  }

  // acc[b] in lane (j, g), component v: out[row j][4g + v] (partial over this wave's units)
  constexpr int F = 256 / NW, S = 64 / F, PPL = NW / S;
  static_assert(F >= 1 && F <= 64 && 64 % F == 0 && NW % S == 0, "out reduction split");
  const float* partf = reinterpret_cast<const float*>(&part[0][0]);
#pragma unroll
  for (int b = 0; b < RBW; ++b) {
    if (rb0 + b >= nrb) break;  // uniform
    part[w][lane] = acc[b];
    __syncthreads();
    const int f = lane % F, pg = lane / F;
    const int fi = w * F + f;
    const int src = (fi >> 2) & 63, v = fi & 3;
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < PPL; ++i) s += partf[((pg * PPL + i) * 64 + src) * 4 + v];
#pragma unroll
    for (int m = F; m < 64; m <<= 1) s += __shfl_xor(s, m);
    const int row = (rb0 + b) * 16 + (src & 15);
    const int col = 4 * (src >> 4) + v;
    if (pg == 0 && row < M) {
      if constexpr (OUT_F32) reinterpret_cast<float*>(out)[(int64_t)row * ldo + col] = s;
      else reinterpret_cast<uint16_t*>(out)[(int64_t)row * ldo + col] = (uint16_t)pack_bf16x2(s, 0.f);
    }
    __syncthreads();
  }
}

// ------------------------------------------------------------------ transposed dequant-GEMM
// part[rg][n][k] = sum over the rows m of row group rg of x_hat[m][n] * gm[m][k] (x_hat =
// bf16(decode), k < 16 KT).  Grid: (column groups of UPW units) x (row groups of bpg 16-row
// blocks) in one XCD-aware dimension; wave w of a workgroup takes the group's blocks w, w + NW,
// ... over all UPW units, through a ring of PD register slots (loads of later blocks in flight
// while one is computed).
// Every MFMA operand keeps K along a lane's registers, and the reduction here runs over rows.
// So the reconstruction is made directly in that layout: with L as the A operand and V as the
// B operand, the low-rank MFMA's output holds, in lane (j, g), rows 4g .. 4g+3 of one column
// (the C operand, code * scale + zero, is built in the same layout from four rows' codes and
// qparams).  Packed to bf16 it is the B operand of the product with gm^T (gm's rows transposed
// once per block by an identity MFMA), whose accumulator holds, in lane (j, g), 4 consecutive k
// of that column.  The columns of the workgroup's span (UPW G per plane) are dealt to lanes in
// byte order: lane j reads the BPL = UPW G / 16 consecutive code bytes BPL j .. of each of its
// rows, and byte t of them is its column in tile t (TT = BPL tiles per plane).  The NW waves'
// accumulators are summed through LDS in wave order (deterministic) and leave as 16-byte rows.
template <int BITS, int G, int R, int KT, int NW, int UPW, int PD, int NBM>
__global__ __launch_bounds__(NW * 64) void k_dequant_gemm_t(
    const uint8_t* __restrict__ codes, int64_t ldc, const uint16_t* __restrict__ qparams, int64_t ldq,
    const uint16_t* __restrict__ Lin, int64_t ldl, const uint16_t* __restrict__ V, int M, int N,
    const uint16_t* __restrict__ gm, int64_t ldg, float* __restrict__ part, int bpg, int ncg, bool xcd_map) {
  constexpr int NP = 8 / BITS, RT = R > 0 ? R / 16 : 1;
  constexpr int SPAN = UPW * G;             // columns of one plane in the workgroup's span
  constexpr int BPL = SPAN / 16, TT = BPL;  // code bytes per lane and row; tiles per plane
  constexpr int DW = BPL / 4;               // code dwords per lane and row
  constexpr int NACC = NP * TT * KT;        // f32x4 accumulators per lane
  constexpr int CH = NACC < 8 ? NACC : 8;   // accumulators per LDS round
  static_assert(NACC % CH == 0, "reduction rounds");
  static_assert(BPL % 4 == 0 && BPL <= 16 && G % BPL == 0, "a lane's bytes are whole dwords of one unit");
  static_assert(NP <= 2, "4- or 8-bit codes");
  __shared__ f32x4 red[NW][CH][64];
  const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int j = lane & 15, g = lane >> 4;
  const int nrb = (M + 15) / 16;
  // workgroup -> (column group, row group).  Workgroups go to the 8 XCDs round-robin by id, and
  // every column group of a row group reads the same qparams, L and g lines: with xcd_map the
  // ids of one XCD (id % 8) take whole row groups, so each line is fetched into one XCD's L2
  // only (without it, 8 L2s fetch it: 2.2x the algorithmic HBM bytes at the north-star shape)
  const int id = blockIdx.x;
  // (the divisions run on the vector unit: readfirstlane brings the uniform results back to
  // scalar registers, so that all block addressing below stays scalar)
  const int cgi = __builtin_amdgcn_readfirstlane(xcd_map ? (id >> 3) % ncg : id % ncg);
  const int rgi = __builtin_amdgcn_readfirstlane(xcd_map ? (id & 7) + 8 * ((id >> 3) / ncg) : id / ncg);
  const int u0 = cgi * UPW;
  const int ul = u0 + (BPL * j) / G;        // the unit of lane j's columns
  const int rb_lo = rgi * bpg, rb_hi = min(rb_lo + bpg, nrb);
  const int KO = 16 * KT;  // gm columns and part row length
  const u32x2 ident = identity_bop(j, g);

  // B operands of the low-rank term: lane (j, g) holds V[column of tile t][ranks 4g ..] (and
  // 16 + 4g .. at rank 32, the K order of residual_unit)
  u32x2 vop[NP][TT][RT];
  if constexpr (R > 0) {
#pragma unroll
    for (int p = 0; p < NP; ++p)
#pragma unroll
      for (int t = 0; t < TT; ++t)
#pragma unroll
        for (int r = 0; r < RT; ++r)
          vop[p][t][r] = ld8(V + (int64_t)(p * (N / NP) + u0 * G + BPL * j + t) * R + 16 * r + 4 * g);
  }
  f32x4 acc[NACC];
#pragma unroll
  for (int a = 0; a < NACC; ++a) acc[a] = zero4();

  struct Blk {
    uint32_t cw[4][DW];  // rows 4g + v: code dwords (bytes BPL j .. of the span)
    uint32_t qp[4][NP];  // rows 4g + v: (scale, zero) of each plane of the lane's unit
    u32x2 lop[RT];       // row j: L ranks 4g .. (A operand)
    u32x2 gop[KT];       // row j: gm columns 16t + 4g ..
  };
  // A block's loads: 32-bit lane offsets from the block's wave-uniform bases.  Row clamping
  // (rows past M repeat the last row) is a min on the offsets, min(r, lim) * ld = min(r * ld,
  // lim * ld), with the lane's r * ld computed once.  lim is the last present row of the block,
  // at most 15, so with row strides below 2^24 bytes (checked by the launch) every offset,
  // lim * ld included, stays below 2^28.
  const uint32_t ldc1 = (uint32_t)ldc, ldq2 = (uint32_t)ldq * 2, ldl2 = (uint32_t)ldl * 2, ldg2 = (uint32_t)ldg * 2;
  uint32_t coff[4], qoff[4];
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    coff[v] = (uint32_t)(4 * g + v) * ldc1;
    qoff[v] = (uint32_t)(4 * g + v) * ldq2;
  }
  const uint32_t loff = (uint32_t)j * ldl2, goff = (uint32_t)j * ldg2;
  const uint32_t cl = (uint32_t)(BPL * j), ql = (uint32_t)(ul * NP * 4), rl = (uint32_t)(8 * g);
  auto load = [&](int rb, Blk& d) {
    const int r0 = rb * 16;                  // wave-uniform
    const uint32_t lim = (uint32_t)min(M - 1 - r0, 15);
    const uint8_t* cbase = codes + (int64_t)r0 * ldc + u0 * G;
    const uint8_t* qbase = reinterpret_cast<const uint8_t*>(qparams + (int64_t)r0 * ldq);
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const uint8_t* cp = cbase + (min(coff[v], lim * ldc1) + cl);
      if constexpr (DW == 4) {
        const u32x4 c = ld16_stream(cp);
#pragma unroll
        for (int e = 0; e < 4; ++e) d.cw[v][e] = c[e];
      } else if constexpr (DW == 2) {
        const u32x2 c = ld8_stream(cp);
        d.cw[v][0] = c[0];
        d.cw[v][1] = c[1];
      } else {
        d.cw[v][0] = ld4(cp);
      }
      const uint8_t* qq = qbase + (min(qoff[v], lim * ldq2) + ql);
      if constexpr (NP == 2) {
        const u32x2 q = ld8(qq);
        d.qp[v][0] = q[0];
        d.qp[v][1] = q[1];
      } else {
        d.qp[v][0] = ld4(qq);
      }
    }
    if constexpr (R > 0) {
      const uint8_t* lbase = reinterpret_cast<const uint8_t*>(Lin + (int64_t)r0 * ldl);
      const uint32_t lo = min(loff, lim * ldl2) + rl;
#pragma unroll
      for (int t = 0; t < RT; ++t) d.lop[t] = ld8(lbase + (lo + 32 * t));
    }
    const uint8_t* gbase = reinterpret_cast<const uint8_t*>(gm + (int64_t)r0 * ldg);
    const uint32_t go = min(goff, lim * ldg2) + rl;
#pragma unroll
    for (int t = 0; t < KT; ++t) d.gop[t] = ld8(gbase + (go + 32 * t));
  };

  // one block's contribution (none for a block past the wave's last: blive false)
  auto process = [&](const Blk& cur, int rb, bool blive) {
    // g^T operands: rows past M contribute nothing (their clamped x_hat is finite)
    const bool live = blive && rb * 16 + j < M;
    u32x2 a2[KT];
#pragma unroll
    for (int t = 0; t < KT; ++t) {
      const u32x2 gv = live ? cur.gop[t] : u32x2{0u, 0u};
      const f32x4 d = mfma_16x16x16(gv, ident, zero4());  // lane (j, g): gm[4g + v][16t + j]
      a2[t] = u32x2{pack_bf16x2_exact(d[0], d[1]), pack_bf16x2_exact(d[2], d[3])};
    }
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      float sf[4], zf[4];
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        sf[v] = f16_val(cur.qp[v][p] & 0xffffu);
        zf[v] = f16_val(cur.qp[v][p] >> 16);
      }
#pragma unroll
      for (int dw = 0; dw < DW; ++dw) {
        uint32_t wq[4];  // row 4g + v: plane p's codes of tiles 4 dw .. 4 dw + 3, one per byte
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const uint32_t wd = cur.cw[v][dw];
          wq[v] = NP == 1 ? wd : ((wd >> (BITS * p)) & (0x01010101u * ((1u << BITS) - 1u)));
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int t = 4 * dw + e;
          f32x4 x;
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            const float q = e == 0 ? ubyte_f32<0>(wq[v]) : e == 1 ? ubyte_f32<1>(wq[v]) : e == 2 ? ubyte_f32<2>(wq[v])
                                                                                             : ubyte_f32<3>(wq[v]);
            x[v] = __builtin_fmaf(q, sf[v], zf[v]);
          }
          // + (L V^T)[4g + v][column], rounded once with the C operand above
          if constexpr (R == 16) {
            x = mfma_16x16x16(cur.lop[0], vop[p][t][0], x);
          } else if constexpr (R == 32) {
            x = mfma_16x16x32(u32x4{cur.lop[0][0], cur.lop[0][1], cur.lop[1][0], cur.lop[1][1]},
                              u32x4{vop[p][t][0][0], vop[p][t][0][1], vop[p][t][1][0], vop[p][t][1][1]}, x);
          }
          const u32x2 xb = u32x2{pack_bf16x2(x[0], x[1]), pack_bf16x2(x[2], x[3])};  // x_hat rows 4g + v
#pragma unroll
          for (int kt = 0; kt < KT; ++kt) {
            f32x4& c = acc[(p * TT + t) * KT + kt];
            c = mfma_16x16x16(a2[kt], xb, c);
          }
        }
      }
    }
  };

  // The wave's blocks rb_lo + w + i NW, i < nb, in chunks of NBM blocks.  A chunk is straight-
  // line code without branches: its first PD blocks' loads go out together, and each block's
  // slot is refilled with the block PD later right after it is used, so every wait counts
  // exactly the loads issued after the slot's own.  (A loop over the ring makes the compiler
  // merge the slot states of the loop entry and back edge, and a branch around a block lets it
  // sink that block's loads to their use; either way a block would wait for nearly every load
  // in flight.)  Loads are clamped to the group's last block; blocks past the wave's last are
  // computed with a zero gm operand and add nothing.  The launch picks NBM to cover the waves'
  // block counts where it can.
  const int nb = rb_lo + w < rb_hi ? (rb_hi - rb_lo - w + NW - 1) / NW : 0;
  const int last = rb_hi - 1;
  for (int c0 = 0; c0 < nb; c0 += NBM) {  // wave-uniform
    Blk ring[PD];
#pragma unroll
    for (int sl = 0; sl < PD; ++sl) load(min(rb_lo + w + (c0 + sl) * NW, last), ring[sl]);
    __builtin_amdgcn_sched_barrier(0);
    static_for<0, NBM>([&](auto ic) {
      constexpr int i = decltype(ic)::value;
      const int rb = rb_lo + w + (c0 + i) * NW;
      process(ring[i % PD], rb, c0 + i < nb);
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (i + PD < NBM) load(min(rb + PD * NW, last), ring[i % PD]);
      __builtin_amdgcn_sched_barrier(0);
    });
  }

  // acc[(p TT + t) KT + kt] in lane (j, g), component v: column
  // n = p N/NP + u0 G + BPL j + t, k = 16 kt + 4g + v
  float* partg = part + (int64_t)rgi * N * KO;
#pragma unroll
  for (int c0 = 0; c0 < NACC; c0 += CH) {
#pragma unroll
    for (int c = 0; c < CH; ++c) red[w][c][lane] = acc[c0 + c];
    __syncthreads();
    for (int e = threadIdx.x; e < CH * 64; e += NW * 64) {
      const int c = e >> 6, ln = e & 63;
      f32x4 s = red[0][c][ln];
#pragma unroll
      for (int ww = 1; ww < NW; ++ww) {
        const f32x4 o = red[ww][c][ln];
        s[0] += o[0];
        s[1] += o[1];
        s[2] += o[2];
        s[3] += o[3];
      }
      const int a = c0 + c, kt = a % KT, t = (a / KT) % TT, p = a / (KT * TT);
      const int jj = ln & 15, gg = ln >> 4;
      const int n = p * (N / NP) + u0 * G + BPL * jj + t;
      st16(partg + (int64_t)n * KO + 16 * kt + 4 * gg,
           u32x4{__float_as_uint(s[0]), __float_as_uint(s[1]), __float_as_uint(s[2]), __float_as_uint(s[3])});
    }
    __syncthreads();
  }
}

// Transposed dequant-GEMM on the rotated format: part[rg][n][k] = sum over the rows m of row
// group rg of x_hat[m][n] * gm[m][k], x_hat = bf16(WHT128(bf16(Y'))) blockwise as the rotated
// decode returns it.  A workgroup takes one 128-column rotation block of each plane (the
// 128 / G units cgi * 128 / G ..) over one row group; its waves take whole 16-row blocks each,
// with no LDS and no barrier until the final reduction.  Per block a lane reconstructs Y' of
// row j at 32 columns (the units' G/4-column quarters, as in the decode), gathered by
// rot_gather_128 into the data operand of the rotation.  The rotation's MFMAs run with the data
// as the A operand and the sign matrix as the B operand: the transposed product of the
// decode's wht128_lds, with the same operand registers and the same sums, so x_hat is the
// decode's bit for bit.  Their output holds, in lane (j, g), rows 4g .. 4g+3 of one rotated
// column: K along the registers, the layout of the product with gm (gm's rows transposed by an
// identity MFMA as in k_dequant_gemm_t), with no transpose of x_hat.  rot_col gives the column
// of output tile q in lane j (the row index of wht128_lds's output tile).  With two planes and
// large accumulators a wave takes one plane (PPW = 1; waves w and w + 1 read the same code
// bytes).  The waves of a plane are summed through LDS in wave order and leave as 16-byte rows.
__device__ __forceinline__ int rot_col(int j, int q) { return (j & 3) + 4 * q + 32 * (j >> 2); }

template <int BITS, int G, int R, int KT, int NW, int PPW, int PD, int NBM>
__global__ __launch_bounds__(NW * 64) void k_dequant_gemm_t_rot(
    const uint8_t* __restrict__ codes, int64_t ldc, const uint16_t* __restrict__ qparams, int64_t ldq,
    const uint16_t* __restrict__ Lin, int64_t ldl, const uint16_t* __restrict__ V, int M, int N,
    const uint16_t* __restrict__ gm, int64_t ldg, float* __restrict__ part, int bpg, int ncg, bool xcd_map) {
  constexpr int NP = 8 / BITS, RT = R > 0 ? R / 16 : 1, E = G / 4;
  constexpr int U = 128 / G;                // units of one rotation block
  constexpr int NG = NP / PPW;              // plane groups: waves w, w + NG, ... share a plane set
  constexpr int WB = NW / NG;               // waves per plane group
  constexpr int NACC = PPW * 8 * KT;        // f32x4 accumulators per lane
  constexpr int CH = NACC < 8 ? NACC : 8;   // accumulators per LDS round
  static_assert(NP % PPW == 0 && NW % NG == 0 && NACC % CH == 0, "plane groups and reduction rounds");
  __shared__ f32x4 red[NW][CH][64];
  const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int j = lane & 15, g = lane >> 4;
  const int grp = w % NG, wb = w / NG;      // plane group; the wave's place among the group's waves
  const int nrb = (M + 15) / 16;
  // workgroup -> (rotation block, row group), XCD-aware as in k_dequant_gemm_t
  const int id = blockIdx.x;
  const int cgi = __builtin_amdgcn_readfirstlane(xcd_map ? (id >> 3) % ncg : id % ncg);
  const int rgi = __builtin_amdgcn_readfirstlane(xcd_map ? (id & 7) + 8 * ((id >> 3) / ncg) : id / ncg);
  const int u0 = cgi * U;
  const int rb_lo = rgi * bpg, rb_hi = min(rb_lo + bpg, nrb);
  const int KO = 16 * KT;
  const u32x2 ident = identity_bop(j, g);
  u32x4 wop[2][2];
#pragma unroll
  for (int q0 = 0; q0 < 2; ++q0)
#pragma unroll
    for (int n = 0; n < 2; ++n) wop[q0][n] = wht_base_operand(j, rot_sign_group<G>(g), q0, n != 0);

  // reconstruction operands of the wave's planes (the same for every block)
  u32x2 vop[PPW][U][G / 16][RT];
  if constexpr (R > 0) {
#pragma unroll
    for (int pi = 0; pi < PPW; ++pi)
#pragma unroll
      for (int ul = 0; ul < U; ++ul) load_vops<G, R>(V, unit_base(grp * PPW + pi, u0 + ul, N, NP, G), j, g, vop[pi][ul]);
  }
  f32x4 acc[NACC];
#pragma unroll
  for (int a = 0; a < NACC; ++a) acc[a] = zero4();

  struct Blk {
    u32x4 cb[U][G / 64];  // row j: the lane's G/4 code bytes of each unit
    uint32_t qp[U][PPW];  // row j: (scale, zero) of the wave's planes of each unit
    u32x2 lop[RT];        // row j: L ranks 4g .. (B operand of the reconstruction)
    u32x2 gop[KT];        // row j: gm columns 16t + 4g ..
  };
  // 32-bit lane offsets from the block's wave-uniform bases, rows past M clamped to the last
  // (min(r, lim) * ld = min(r * ld, lim * ld)); strides below 2^24 bytes are checked by the launch
  const uint32_t ldc1 = (uint32_t)ldc, ldq2 = (uint32_t)ldq * 2, ldl2 = (uint32_t)ldl * 2, ldg2 = (uint32_t)ldg * 2;
  const uint32_t coff = (uint32_t)j * ldc1, qoff = (uint32_t)j * ldq2, loff = (uint32_t)j * ldl2,
                 goff = (uint32_t)j * ldg2;
  const uint32_t rl = (uint32_t)(8 * g);
  auto load = [&](int rb, Blk& d) __attribute__((always_inline)) {
    const int r0 = rb * 16;  // wave-uniform
    const uint32_t lim = (uint32_t)min(M - 1 - r0, 15);
    const uint8_t* cbase = codes + (int64_t)r0 * ldc + u0 * G;
    const uint8_t* qbase = reinterpret_cast<const uint8_t*>(qparams + (int64_t)r0 * ldq) + u0 * NP * 4;
    const uint32_t co = min(coff, lim * ldc1) + (uint32_t)(E * g), qo = min(qoff, lim * ldq2);
#pragma unroll
    for (int ul = 0; ul < U; ++ul) {
#pragma unroll
      for (int i = 0; i < G / 64; ++i) d.cb[ul][i] = ld16_stream(cbase + (co + (uint32_t)(ul * G + 16 * i)));
      if constexpr (PPW == 2) {
        const u32x2 q = ld8(qbase + (qo + (uint32_t)(ul * 8)));
        d.qp[ul][0] = q[0];
        d.qp[ul][1] = q[1];
      } else {
        d.qp[ul][0] = ld4(qbase + (qo + (uint32_t)(ul * NP * 4 + grp * 4)));
      }
    }
    if constexpr (R > 0) {
      const uint8_t* lbase = reinterpret_cast<const uint8_t*>(Lin + (int64_t)r0 * ldl);
      const uint32_t lo = min(loff, lim * ldl2) + rl;
#pragma unroll
      for (int t = 0; t < RT; ++t) d.lop[t] = ld8(lbase + (lo + 32 * t));
    }
    const uint8_t* gbase = reinterpret_cast<const uint8_t*>(gm + (int64_t)r0 * ldg);
    const uint32_t go = min(goff, lim * ldg2) + rl;
#pragma unroll
    for (int t = 0; t < KT; ++t) d.gop[t] = ld8(gbase + (go + 32 * t));
  };

  const float kScale = 0.08838834764831845f;  // fp32(1/sqrt(128)), as in wht128_lds
  auto process = [&](const Blk& cur, int rb, bool blive) __attribute__((always_inline)) {
    // g^T operands: rows past M contribute nothing (their clamped x_hat is finite)
    const bool live = blive && rb * 16 + j < M;
    u32x2 a2[KT];
#pragma unroll
    for (int t = 0; t < KT; ++t) {
      const u32x2 gv = live ? cur.gop[t] : u32x2{0u, 0u};
      const f32x4 d = mfma_16x16x16(gv, ident, zero4());  // lane (j, g): gm[4g + v][16t + j]
      a2[t] = u32x2{pack_bf16x2_exact(d[0], d[1]), pack_bf16x2_exact(d[2], d[3])};
    }
#pragma unroll
    for (int pi = 0; pi < PPW; ++pi) {
      const int p = grp * PPW + pi;
      float xh[32];  // row j: Y' at the lane's E columns of each unit
#pragma unroll
      for (int ul = 0; ul < U; ++ul) reconstruct_plane<BITS, G, R>(cur.cb[ul], cur.qp[ul][pi], p, vop[pi][ul], cur.lop, xh + E * ul);
      u32x4 xv[4];
      rot_gather_128<G>(xh, xv);
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        f32x4 y = zero4();
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const int flip = (((q >> 1) & c & 1) ^ ((q >> 2) & (c >> 1) & 1));
          y = mfma_16x16x32(xv[c], wop[q & 1][flip], y);
        }
        // x_hat rows 4g + v of column rot_col(j, q)
        const u32x2 xq = u32x2{pack_bf16x2(y[0] * kScale, y[1] * kScale), pack_bf16x2(y[2] * kScale, y[3] * kScale)};
#pragma unroll
        for (int kt = 0; kt < KT; ++kt) {
          f32x4& c = acc[(pi * 8 + q) * KT + kt];
          c = mfma_16x16x16(a2[kt], xq, c);
        }
      }
    }
  };

  // the wave's blocks rb_lo + wb + i WB, i < nb, in straight-line chunks of NBM blocks with a
  // ring of PD slots (as in k_dequant_gemm_t)
  const int nb = rb_lo + wb < rb_hi ? (rb_hi - rb_lo - wb + WB - 1) / WB : 0;
  const int last = rb_hi - 1;
  for (int c0 = 0; c0 < nb; c0 += NBM) {  // wave-uniform
    Blk ring[PD];
#pragma unroll
    for (int sl = 0; sl < PD; ++sl) load(min(rb_lo + wb + (c0 + sl) * WB, last), ring[sl]);
    __builtin_amdgcn_sched_barrier(0);
    static_for<0, NBM>([&](auto ic) {
      constexpr int i = decltype(ic)::value;
      const int rb = rb_lo + wb + (c0 + i) * WB;
      process(ring[i % PD], rb, c0 + i < nb);
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (i + PD < NBM) load(min(rb + PD * WB, last), ring[i % PD]);
      __builtin_amdgcn_sched_barrier(0);
    });
  }

  // acc[(pi 8 + q) KT + kt] in lane (j, g), component v: column
  // n = p N/NP + u0 G + rot_col(j, q), k = 16 kt + 4g + v (p = grp PPW + pi)
  float* partg = part + (int64_t)rgi * N * KO;
#pragma unroll
  for (int c0 = 0; c0 < NACC; c0 += CH) {
#pragma unroll
    for (int c = 0; c < CH; ++c) red[w][c][lane] = acc[c0 + c];
    __syncthreads();
    for (int e = threadIdx.x; e < NG * CH * 64; e += NW * 64) {
      const int eg = e / (CH * 64), c = (e >> 6) % CH, ln = e & 63;
      f32x4 s = red[eg][c][ln];
#pragma unroll
      for (int i = 1; i < WB; ++i) {
        const f32x4 o = red[eg + NG * i][c][ln];
        s[0] += o[0];
        s[1] += o[1];
        s[2] += o[2];
        s[3] += o[3];
      }
      const int a = c0 + c, kt = a % KT, q = (a / KT) % 8, p = eg * PPW + a / (8 * KT);
      const int jj = ln & 15, gg = ln >> 4;
      const int n = p * (N / NP) + u0 * G + rot_col(jj, q);
      st16(partg + (int64_t)n * KO + 16 * kt + 4 * gg,
           u32x4{__float_as_uint(s[0]), __float_as_uint(s[1]), __float_as_uint(s[2]), __float_as_uint(s[3])});
    }
    __syncthreads();
  }
}

// Outlier channels in dequant_gemm_t: x_hat[:, idx[k]] = bf16(side[:, k]), so output row idx[k]
// is sum over the rows of bf16(side[m, k]) * G[m, :].  One workgroup per channel overwrites that
// row after the main kernels (fp32 sums, a block reduction in a fixed order).
template <int KO, bool OUT_F32>
__global__ __launch_bounds__(256) void k_side_gemm_t(const uint16_t* __restrict__ side, int64_t ldside, int M, int N,
                                                     const int32_t* __restrict__ oidx, const uint16_t* __restrict__ G,
                                                     int64_t ldg, void* __restrict__ out, int64_t ldo) {
  __shared__ float red[KO][256];
  const int k = blockIdx.x, c = oidx[k];
  if (c < 0 || c >= N) return;  // whole workgroup
  float acc[KO];
#pragma unroll
  for (int q = 0; q < KO; ++q) acc[q] = 0.f;
  for (int m = threadIdx.x; m < M; m += 256) {
    const float sv = __uint_as_float(pack_bf16x2(f16_val(side[(int64_t)m * ldside + k]), 0.f) << 16);  // bf16(side)
#pragma unroll
    for (int q = 0; q < KO; q += 4) {
      const u32x2 gv = ld8(G + (int64_t)m * ldg + q);
      acc[q + 0] = __builtin_fmaf(sv, __uint_as_float(gv[0] << 16), acc[q + 0]);
      acc[q + 1] = __builtin_fmaf(sv, __uint_as_float(gv[0] & 0xffff0000u), acc[q + 1]);
      acc[q + 2] = __builtin_fmaf(sv, __uint_as_float(gv[1] << 16), acc[q + 2]);
      acc[q + 3] = __builtin_fmaf(sv, __uint_as_float(gv[1] & 0xffff0000u), acc[q + 3]);
    }
  }
#pragma unroll
  for (int q = 0; q < KO; ++q) red[q][threadIdx.x] = acc[q];
  __syncthreads();
  if (threadIdx.x < KO) {
    float sum = 0.f;
    for (int i = 0; i < 256; ++i) sum += red[threadIdx.x][i];
    if constexpr (OUT_F32) reinterpret_cast<float*>(out)[(int64_t)c * ldo + threadIdx.x] = sum;
    else reinterpret_cast<uint16_t*>(out)[(int64_t)c * ldo + threadIdx.x] = (uint16_t)pack_bf16x2(sum, 0.f);
  }
}

static int side_gemm_t(const lrq_tensors* t, const void* g, int64_t ldg, int n_out, void* out, int64_t ldo, bool f32,
                       hipStream_t s) {
  if (t->n_outlier == 0) return LRQ_OK;
  const dim3 grid((unsigned)t->n_outlier), block(256);
  const int M = (int)t->rows, N = (int)t->hidden;
  const auto* sd = (const uint16_t*)t->side;
  const auto* gg = (const uint16_t*)g;
  switch (n_out * 2 + (f32 ? 1 : 0)) {
    case 16 * 2 + 1: return launch((k_side_gemm_t<16, true>), grid, block, 0, s, sd, t->ld_side, M, N, t->outlier_idx, gg, ldg, out, ldo);
    case 16 * 2: return launch((k_side_gemm_t<16, false>), grid, block, 0, s, sd, t->ld_side, M, N, t->outlier_idx, gg, ldg, out, ldo);
    case 32 * 2 + 1: return launch((k_side_gemm_t<32, true>), grid, block, 0, s, sd, t->ld_side, M, N, t->outlier_idx, gg, ldg, out, ldo);
    case 32 * 2: return launch((k_side_gemm_t<32, false>), grid, block, 0, s, sd, t->ld_side, M, N, t->outlier_idx, gg, ldg, out, ldo);
    default: return LRQ_ERR_UNSUPPORTED;
  }
}

// out[n][k] = sum over the rg row groups of part[.][n][k] in group order (fp32), for nk = N KO
// entries; 4 consecutive k per thread.  rg == 0 (no rows) writes zeros.
template <bool OUT_F32>
__global__ __launch_bounds__(256) void k_sum_parts(const float* __restrict__ part, int rg, int64_t nk, int KO,
                                                   void* __restrict__ out, int64_t ldo) {
  const int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
  if (i >= nk) return;
  float s[4] = {0.f, 0.f, 0.f, 0.f};
  // 8 groups' loads in flight at a time, summed in group order
  int r = 0;
  for (; r + 8 <= rg; r += 8) {
    u32x4 v[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) v[k] = ld16(part + (int64_t)(r + k) * nk + i);
#pragma unroll
    for (int k = 0; k < 8; ++k)
#pragma unroll
      for (int e = 0; e < 4; ++e) s[e] += __uint_as_float(v[k][e]);
  }
  for (; r < rg; ++r) {
    const u32x4 v = ld16(part + (int64_t)r * nk + i);
#pragma unroll
    for (int e = 0; e < 4; ++e) s[e] += __uint_as_float(v[e]);
  }
  const int64_t n = i / KO, k = i % KO;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    if constexpr (OUT_F32) reinterpret_cast<float*>(out)[n * ldo + k + e] = s[e];
    else reinterpret_cast<uint16_t*>(out)[n * ldo + k + e] = (uint16_t)pack_bf16x2(s[e], 0.f);
  }
}

// ------------------------------------------------------------------ host side
template <int BITS, int G, int R, int NW, int UPW>
static int softmax_launch(const lrq_tensors* t, const void* dp, int64_t lddp, void* ds, int64_t ldds, hipStream_t s) {
  constexpr int RBW = 2;
  const int M = (int)t->rows, N = (int)t->hidden;
  const int nrb = (M + 15) / 16;
  LRQ_TRY(launch((k_softmax_bwd<BITS, G, R, NW, UPW, RBW>), dim3((nrb + RBW - 1) / RBW), dim3(NW * 64), 0, s,
                     (const uint8_t*)t->codes, t->ld_codes, (const uint16_t*)t->qparams, t->ld_qp,
                     (const uint16_t*)t->L, t->ld_L, (const uint16_t*)t->V, M, N, (const uint16_t*)dp, lddp,
                     (uint16_t*)ds, ldds));
  return LRQ_OK;
}

template <int BITS, int G, int R, int NW>
static int softmax_rows_launch(const lrq_tensors* t, const void* dp, int64_t lddp, void* ds, int64_t ldds,
                               hipStream_t s) {
  using St = SmxTile<BITS, G, NW>;
  const int M = (int)t->rows, N = (int)t->hidden;
  const int nrb = (M + 15) / 16;
  const int per_cu = std::max(1, std::min(4, (int)((160 * 1024) / St::LDS)));
  const int wgs = std::max(1, std::min(nrb, cu_count() * per_cu));
  const int rbw = (nrb + wgs - 1) / wgs;
  auto kern = k_softmax_rows<BITS, G, R, NW>;
  hipError_t e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)St::LDS);
  if (e != hipSuccess) return (int)e;
  LRQ_TRY(launch(kern, dim3((nrb + rbw - 1) / rbw), dim3(NW * 64), St::LDS, s, (const uint8_t*)t->codes,
                     t->ld_codes, (const uint16_t*)t->qparams, t->ld_qp, (const uint16_t*)t->L, t->ld_L,
                     (const uint16_t*)t->V, M, N, (const uint16_t*)dp, lddp, (uint16_t*)ds, ldds, rbw));
  return LRQ_OK;
}

// Any other row width: the two-sweep kernel, about four workgroups per CU.
template <int BITS, int G, int R>
static int softmax_2s_launch(const lrq_tensors* t, const void* dp, int64_t lddp, void* ds, int64_t ldds,
                             hipStream_t s) {
  constexpr int NW = 8;
  // units held in registers per wave: four units of 128 columns, two of 256 (rank 32: none)
  constexpr int HOLD = R > 16 ? 0 : G * (8 / BITS) <= 128 ? 4 : 2;
  using Sm = Smx2s<BITS, G, R, NW, HOLD>;
  const int M = (int)t->rows, N = (int)t->hidden;
  const int64_t units = t->hidden / ((int64_t)G * (8 / BITS));
  const int nrb = (M + 15) / 16;
  const int wgs = std::max(1, std::min(nrb, cu_count() * 4));
  const int rbw = (nrb + wgs - 1) / wgs;
  auto go = [&](auto kern, size_t shm) {
    if (shm > 64 * 1024) {
      const hipError_t e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)shm);
      if (e != hipSuccess) return (int)e;
    }
    return launch(kern, dim3((nrb + rbw - 1) / rbw), dim3(NW * 64), shm, s, (const uint8_t*)t->codes, t->ld_codes,
                  (const uint16_t*)t->qparams, t->ld_qp, (const uint16_t*)t->L, t->ld_L, (const uint16_t*)t->V, M, N,
                  (const uint16_t*)dp, lddp, (uint16_t*)ds, ldds, rbw);
  };
  if constexpr (HOLD > 0) {
    if (units >= NW && units <= (int64_t)NW * HOLD) return go(k_softmax_2s<BITS, G, R, NW, HOLD>, Sm::LDS);
  }
  return go(k_softmax_2s<BITS, G, R, NW, 0>, 0);
}

// Rotated format (planes of whole rotation blocks, no outlier channels): the rotated two-sweep
// kernel, about four workgroups per CU.
template <int BITS, int G, int R>
static int softmax_rot_launch(const lrq_tensors* t, const void* dp, int64_t lddp, void* ds, int64_t ldds,
                              hipStream_t s) {
  constexpr int NW = 8;
  // items held in registers per wave: two (rank 32: none)
  constexpr int HOLD = R > 16 ? 0 : 2;
  const int M = (int)t->rows, N = (int)t->hidden;
  const int64_t items = t->hidden / ((8 / BITS) * 128);
  const int nrb = (M + 15) / 16;
  const int wgs = std::max(1, std::min(nrb, cu_count() * 4));
  const int rbw = (nrb + wgs - 1) / wgs;
  auto go = [&](auto kern, size_t shm) {
    if (shm > 64 * 1024) {
      const hipError_t e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)shm);
      if (e != hipSuccess) return (int)e;
    }
    return launch(kern, dim3((nrb + rbw - 1) / rbw), dim3(NW * 64), shm, s, (const uint8_t*)t->codes, t->ld_codes,
                  (const uint16_t*)t->qparams, t->ld_qp, (const uint16_t*)t->L, t->ld_L, (const uint16_t*)t->V, M, N,
                  (const uint16_t*)dp, lddp, (uint16_t*)ds, ldds, rbw);
  };
  if constexpr (HOLD > 0) {
    // one workgroup per CU (the parked V operands and the held inputs allow no second), each
    // walking its row blocks with the next block's inputs in flight
    if (items >= NW && items <= (int64_t)NW * HOLD) {
      const int pw = std::max(1, std::min(nrb, cu_count()));
      const int prbw = (nrb + pw - 1) / pw;
      const size_t shm = SmxRot<BITS, G, R, NW, HOLD>::LDS;
      auto kern = k_softmax_rot<BITS, G, R, NW, HOLD>;
      if (shm > 64 * 1024) {
        const hipError_t e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)shm);
        if (e != hipSuccess) return (int)e;
      }
      return launch(kern, dim3((nrb + prbw - 1) / prbw), dim3(NW * 64), shm, s, (const uint8_t*)t->codes,
                    t->ld_codes, (const uint16_t*)t->qparams, t->ld_qp, (const uint16_t*)t->L, t->ld_L,
                    (const uint16_t*)t->V, M, N, (const uint16_t*)dp, lddp, (uint16_t*)ds, ldds, prbw);
    }
  }
  return go(k_softmax_rot<BITS, G, R, NW, 0>, 0);
}

// One pass needs the whole row in one workgroup: 4, 8 or 16 units (one per wave).  Rows of
// whole 1 KB chunks take the row-persistent kernel; every other width the two-sweep kernel.
template <int BITS, int G, int R>
static int softmax_units(const lrq_tensors* t, const void* dp, int64_t lddp, void* ds, int64_t ldds, hipStream_t s) {
  const int64_t units = t->hidden / ((int64_t)G * (8 / BITS));
  constexpr int UB = G * (8 / BITS) * 2;  // bf16 bytes of one unit of a row
  if ((units == 16 && (16 * UB) % 1024 == 0) || (units == 8 && (8 * UB) % 1024 == 0)) {
    if (units == 16) {
      if constexpr ((16 * UB) % 1024 == 0 && 2 * 16 * (16 * UB + 16) + 1024 <= 160 * 1024)
        return softmax_rows_launch<BITS, G, R, 16>(t, dp, lddp, ds, ldds, s);
    } else {
      if constexpr ((8 * UB) % 1024 == 0 && 2 * 16 * (8 * UB + 16) + 512 <= 160 * 1024)
        return softmax_rows_launch<BITS, G, R, 8>(t, dp, lddp, ds, ldds, s);
    }
  }
  switch (units) {
    case 4: return softmax_launch<BITS, G, R, 4, 1>(t, dp, lddp, ds, ldds, s);
    case 8: return softmax_launch<BITS, G, R, 8, 1>(t, dp, lddp, ds, ldds, s);
    case 16: return softmax_launch<BITS, G, R, 16, 1>(t, dp, lddp, ds, ldds, s);
    default: return softmax_2s_launch<BITS, G, R>(t, dp, lddp, ds, ldds, s);
  }
}

// k_dequant_gemm_t addresses a block's rows by 32-bit offsets (row in block x row stride):
// strides below 2^24 bytes keep them in range.
static bool strides_fit24(const lrq_tensors* t, int64_t ldg_elems) {
  constexpr int64_t kLim = int64_t(1) << 24;
  return t->ld_codes < kLim && t->ld_qp * 2 < kLim && t->ld_L * 2 < kLim && ldg_elems * 2 < kLim;
}

template <int BITS, int G, int R, int NOUT, bool F32, bool OUTL>
static int gemm_launch(const lrq_tensors* t, const void* a, void* out, int64_t ldo, hipStream_t s) {
  // row blocks per workgroup: 4, or 2 where a unit's register slot is large (two slots in flight)
  constexpr int UC = G * (8 / BITS);  // columns of one unit
  constexpr int NW = 8, RBW = (UC >= 256 && NOUT == 32) ? 1 : (UC >= 256 || NOUT == 32 || R == 32) ? 2 : 4;
  // unit slots in flight (one where a slot is large; the outlier mask adds registers to a slot)
  constexpr int SL = (UC >= 256 && R > 0 && (NOUT == 32 || OUTL)) ? 1 : 2;
  const int M = (int)t->rows, N = (int)t->hidden;
  const int nrb = (M + 15) / 16;
  const size_t shm = OUTL ? (size_t)(N / 32) * 4 : 0;
  if constexpr (NOUT == 16 && R <= 16) {
    // units split evenly over the waves: the wave-resident kernel (NU units per wave)
    const int units = N / UC;
    auto wlaunch = [&](auto nu) {
      // one block in flight with the outlier mask (its registers would not fit beside a second)
      constexpr int NU = decltype(nu)::value, WRBW = 4, WSL = OUTL ? 1 : 2;
      LRQ_TRY(launch((k_dequant_gemm_w<BITS, G, R, NW, NU, WRBW, WSL, F32, OUTL>), dim3((nrb + WRBW - 1) / WRBW),
                     dim3(NW * 64), shm, s, (const uint8_t*)t->codes, t->ld_codes, (const uint16_t*)t->qparams,
                     t->ld_qp, (const uint16_t*)t->L, t->ld_L, (const uint16_t*)t->V, M, N, (const uint16_t*)a, out,
                     ldo, t->outlier_idx, (int)t->n_outlier, (const uint16_t*)t->side, t->ld_side));
      return LRQ_OK;
    };
    if (units == NW * 4) return wlaunch(std::integral_constant<int, 4>{});
    if (units == NW * 2) return wlaunch(std::integral_constant<int, 2>{});
    if (units == NW) return wlaunch(std::integral_constant<int, 1>{});
  }
  LRQ_TRY(launch((k_dequant_gemm<BITS, G, R, NOUT, NW, RBW, SL, F32, OUTL>), dim3((nrb + RBW - 1) / RBW),
                 dim3(NW * 64), shm, s, (const uint8_t*)t->codes, t->ld_codes, (const uint16_t*)t->qparams, t->ld_qp,
                 (const uint16_t*)t->L, t->ld_L, (const uint16_t*)t->V, M, N, (const uint16_t*)a, out, ldo,
                 t->outlier_idx, (int)t->n_outlier, (const uint16_t*)t->side, t->ld_side));
  return LRQ_OK;
}

// Rotated format, rotation in registers (k_dequant_gemm_rotr): four row blocks per workgroup
// (two at rank 32, whose V operands would otherwise spill).
template <int BITS, int G, int R, int NOUT, bool F32, bool OUTL>
static int gemm_rotr_launch(const lrq_tensors* t, const void* a, void* out, int64_t ldo, hipStream_t s) {
  constexpr int NP = 8 / BITS, NW = 8, RBW = R == 32 ? 2 : 4;
  if ((t->hidden / NP) % 128 != 0) return LRQ_ERR_UNSUPPORTED;
  const int M = (int)t->rows, N = (int)t->hidden;
  const int nrb = (M + 15) / 16;
  const size_t shm = OUTL ? (size_t)(N / 32) * 4 : 0;
  LRQ_TRY(launch((k_dequant_gemm_rotr<BITS, G, R, NOUT, NW, RBW, F32, OUTL>), dim3((nrb + RBW - 1) / RBW),
                 dim3(NW * 64), shm, s, (const uint8_t*)t->codes, t->ld_codes, (const uint16_t*)t->qparams,
                 t->ld_qp, (const uint16_t*)t->L, t->ld_L, (const uint16_t*)t->V, M, N, (const uint16_t*)a, out, ldo,
                 t->outlier_idx, (int)t->n_outlier, (const uint16_t*)t->side, t->ld_side));
  return LRQ_OK;
}

template <int BITS, int G, int R>
static int gemm_nout(const lrq_tensors* t, const void* a, int n_out, void* out, int64_t ldo, bool f32, hipStream_t s) {
  const bool o = t->n_outlier > 0;
  if (t->flags & LRQ_FLAG_HADAMARD) {
    switch (n_out * 4 + (f32 ? 2 : 0) + (o ? 1 : 0)) {
      case 16 * 4 + 2: return gemm_rotr_launch<BITS, G, R, 16, true, false>(t, a, out, ldo, s);
      case 16 * 4 + 3: return gemm_rotr_launch<BITS, G, R, 16, true, true>(t, a, out, ldo, s);
      case 16 * 4: return gemm_rotr_launch<BITS, G, R, 16, false, false>(t, a, out, ldo, s);
      case 16 * 4 + 1: return gemm_rotr_launch<BITS, G, R, 16, false, true>(t, a, out, ldo, s);
      case 32 * 4 + 2: return gemm_rotr_launch<BITS, G, R, 32, true, false>(t, a, out, ldo, s);
      case 32 * 4 + 3: return gemm_rotr_launch<BITS, G, R, 32, true, true>(t, a, out, ldo, s);
      case 32 * 4: return gemm_rotr_launch<BITS, G, R, 32, false, false>(t, a, out, ldo, s);
      case 32 * 4 + 1: return gemm_rotr_launch<BITS, G, R, 32, false, true>(t, a, out, ldo, s);
      default: return LRQ_ERR_UNSUPPORTED;
    }
  }
  switch (n_out * 4 + (f32 ? 2 : 0) + (o ? 1 : 0)) {
    case 16 * 4 + 2: return gemm_launch<BITS, G, R, 16, true, false>(t, a, out, ldo, s);
    case 16 * 4 + 3: return gemm_launch<BITS, G, R, 16, true, true>(t, a, out, ldo, s);
    case 16 * 4: return gemm_launch<BITS, G, R, 16, false, false>(t, a, out, ldo, s);
    case 16 * 4 + 1: return gemm_launch<BITS, G, R, 16, false, true>(t, a, out, ldo, s);
    case 32 * 4 + 2: return gemm_launch<BITS, G, R, 32, true, false>(t, a, out, ldo, s);
    case 32 * 4 + 3: return gemm_launch<BITS, G, R, 32, true, true>(t, a, out, ldo, s);
    case 32 * 4: return gemm_launch<BITS, G, R, 32, false, false>(t, a, out, ldo, s);
    case 32 * 4 + 1: return gemm_launch<BITS, G, R, 32, false, true>(t, a, out, ldo, s);
    default: return LRQ_ERR_UNSUPPORTED;
  }
}

// Transposed dequant-GEMM.  One unit per workgroup (measured on MI355X at the LoRA shape,
// 16384 x 4096 int4/g64: 17.7 us against 20.7 us with two units per workgroup; a ring of two
// blocks in flight beat three or four, 17.7 against 18.6 / 20.7 us).  Row groups: enough
// workgroups for about one per CU on MI355X (a fixed 256, so the summation order depends only on
// the shapes), at least NW blocks per group.  The workspace holds one fp32 [N, n_out] partial
// per row group.

struct GemmTPlan {
  int upw, cg, rg, bpg;
  int64_t ws_bytes;
};

// k_dequant_gemm_t_rot: planes per wave (one where two planes' accumulators would not fit
// beside the rest) and blocks per straight-line chunk.
constexpr int gemm_t_rot_ppw(int bits, int n_out, int rank) {
  return (8 / bits == 2 && (n_out == 32 || rank == 32)) ? 1 : 8 / bits;
}
constexpr int kGemmTRotChunk = 4;
// k_dequant_gemm_t: accumulators alone take 128 registers (chunks of the ring's two blocks)
constexpr bool gemm_t_big(int bits, int group, int n_out) { return (8 / bits) * (group / 16) * (n_out / 16) > 16; }

// The rotated format's column groups are its rotation blocks (128 columns of each plane).  Row
// groups hold whole chunks per wave where the rows allow (a chunk's blocks past the wave's last
// are computed with a zero g: at 8192 x 5120 the even split gave the waves 9.25 blocks each in
// chunks of 8, so 16 were computed): the blocks per group are the nearest multiple of (waves
// per plane) x (chunk) to the even split.
static GemmTPlan gemm_t_plan(int64_t rows, int64_t hidden, int bits, int group, int rank, int n_out, bool rot) {
  constexpr int NW = 8;
  GemmTPlan pl{};
  const int64_t units = hidden / ((int64_t)group * (8 / bits));
  pl.upw = rot ? 128 / group : 1;
  pl.cg = (int)(units / pl.upw);
  const int64_t nrb = (rows + 15) / 16;
  if (nrb == 0) return pl;  // rg = 0: the sum kernel writes zeros
  const int64_t want = std::max<int64_t>(1, (256 + pl.cg - 1) / pl.cg);
  if (rot) {
    const int64_t q = (int64_t)kGemmTRotChunk * NW / ((8 / bits) / gemm_t_rot_ppw(bits, n_out, rank));
    const int64_t even = (nrb + want - 1) / want;
    pl.bpg = (int)std::max<int64_t>(q, (even + q / 2) / q * q);
  } else {
    const int64_t rg = std::min<int64_t>(want, std::max<int64_t>(1, nrb / NW));
    const int64_t even = (nrb + rg - 1) / rg;
    // the chunk the launch takes for this split (2, 4 or 8 blocks)
    const int64_t q = NW * (gemm_t_big(bits, group, n_out) ? 2 : (even + NW - 1) / NW <= 4 ? 4 : 8);
    pl.bpg = (int)std::max<int64_t>(q, (even + q / 2) / q * q);
  }
  pl.rg = (int)((nrb + pl.bpg - 1) / pl.bpg);
  pl.ws_bytes = (int64_t)pl.rg * hidden * n_out * 4;
  return pl;
}

template <int BITS, int G, int R, int KT, bool F32>
static int gemm_t_run(const lrq_tensors* t, const void* gmat, int64_t ldg, void* out, int64_t ldo, float* ws,
                      const GemmTPlan& pl, hipStream_t s) {
  constexpr int NW = 8;
  constexpr int UPW = 1, PD = 2;  // units per workgroup, blocks in flight per wave
  const int M = (int)t->rows, N = (int)t->hidden;
  if (!strides_fit24(t, ldg)) return LRQ_ERR_UNSUPPORTED;
  if ((t->flags & LRQ_FLAG_HADAMARD) && pl.rg > 0) {
    constexpr int PPW = gemm_t_rot_ppw(BITS, 16 * KT, R);
    LRQ_TRY(launch((k_dequant_gemm_t_rot<BITS, G, R, KT, NW, PPW, PD, kGemmTRotChunk>), dim3(pl.cg * pl.rg),
                   dim3(NW * 64), 0, s,
                   (const uint8_t*)t->codes, t->ld_codes, (const uint16_t*)t->qparams, t->ld_qp, (const uint16_t*)t->L,
                   t->ld_L, (const uint16_t*)t->V, M, N, (const uint16_t*)gmat, ldg, ws, pl.bpg, pl.cg,
                   pl.rg % 8 == 0));
  } else if (pl.rg > 0) {
    // blocks per chunk: the waves' block count ceil(bpg / NW) where it is at most 4, else 8;
    // just the ring's PD blocks where the accumulators alone take 128 registers (the plan makes
    // bpg a multiple of NW x chunk)
    static_assert(UPW == 1, "the plan's chunk rule assumes one unit per workgroup");
    constexpr bool kBig = gemm_t_big(BITS, G, 16 * KT);
    auto kern = kBig ? k_dequant_gemm_t<BITS, G, R, KT, NW, UPW, PD, PD>
                : (pl.bpg + NW - 1) / NW <= 4 ? k_dequant_gemm_t<BITS, G, R, KT, NW, UPW, PD, kBig ? PD : 4>
                                              : k_dequant_gemm_t<BITS, G, R, KT, NW, UPW, PD, kBig ? PD : 8>;
    LRQ_TRY(launch(kern, dim3(pl.cg * pl.rg), dim3(NW * 64), 0, s, (const uint8_t*)t->codes, t->ld_codes,
                   (const uint16_t*)t->qparams, t->ld_qp, (const uint16_t*)t->L, t->ld_L, (const uint16_t*)t->V, M,
                   N, (const uint16_t*)gmat, ldg, ws, pl.bpg, pl.cg, pl.rg % 8 == 0));
  }
  const int64_t nk = (int64_t)N * 16 * KT;
  LRQ_TRY(launch(k_sum_parts<F32>, dim3((unsigned)((nk / 4 + 255) / 256)), dim3(256), 0, s, ws, pl.rg, nk,
                     16 * KT, out, ldo));
  return LRQ_OK;
}

template <int BITS, int G, int R>
static int gemm_t_nout(const lrq_tensors* t, const void* gmat, int64_t ldg, int n_out, void* out, int64_t ldo,
                       bool f32, float* ws, const GemmTPlan& pl, hipStream_t s) {
  switch (n_out * 2 + (f32 ? 1 : 0)) {
    case 16 * 2 + 1: return gemm_t_run<BITS, G, R, 1, true>(t, gmat, ldg, out, ldo, ws, pl, s);
    case 16 * 2: return gemm_t_run<BITS, G, R, 1, false>(t, gmat, ldg, out, ldo, ws, pl, s);
    case 32 * 2 + 1: return gemm_t_run<BITS, G, R, 2, true>(t, gmat, ldg, out, ldo, ws, pl, s);
    case 32 * 2: return gemm_t_run<BITS, G, R, 2, false>(t, gmat, ldg, out, ldo, ws, pl, s);
    default: return LRQ_ERR_UNSUPPORTED;
  }
}

// ---------------------------------------------------------------- allocation-free scratch
// lrq_dequant_gemm_t_noalloc keeps its row-group partials here instead of in a caller
// workspace.  Each GPU holds its own copy of the array at its own address; host code may not
// pass the array's name to a kernel (on the host it is only a stand-in), so the device address
// is looked up once per device with hipGetSymbolAddress and kept.  No partial is read before
// it is written (k_dequant_gemm_t writes every partial of its row group, k_sum_parts reads
// them), so nothing needs clearing between calls.
static __device__ __align__(256) float scratch[LRQ_GEMM_T_SCRATCH_BYTES / sizeof(float)];

static constexpr int kMaxDevices = 64;
static std::mutex g_scratch_mu;
static float* g_scratch_ptr[kMaxDevices];

// The current device's scratch address (looked up on the device's first call), or a positive
// hipError_t.
static int scratch_on_current_device(float** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return (int)e;
  if (dev < 0 || dev >= kMaxDevices) return (int)hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return (int)e;
    if (ptr == nullptr) return (int)hipErrorInvalidSymbol;
    g_scratch_ptr[dev] = static_cast<float*>(ptr);
  }
  *out = g_scratch_ptr[dev];
  return LRQ_OK;
}

#define LRQ_FORMATS(F, ...)                                 \
  switch (format_key(t->bits, t->group, t->rank)) {           \
    case format_key(4, 64, 0): return F<4, 64, 0>(__VA_ARGS__);    \
    case format_key(4, 64, 16): return F<4, 64, 16>(__VA_ARGS__);  \
    case format_key(4, 64, 32): return F<4, 64, 32>(__VA_ARGS__);  \
    case format_key(4, 128, 0): return F<4, 128, 0>(__VA_ARGS__);  \
    case format_key(4, 128, 16): return F<4, 128, 16>(__VA_ARGS__); \
    case format_key(8, 64, 0): return F<8, 64, 0>(__VA_ARGS__);    \
    case format_key(8, 64, 16): return F<8, 64, 16>(__VA_ARGS__);  \
    case format_key(8, 128, 0): return F<8, 128, 0>(__VA_ARGS__);  \
    case format_key(8, 128, 16): return F<8, 128, 16>(__VA_ARGS__); \
    default: return LRQ_ERR_UNSUPPORTED;                      \
  }

}  // namespace lrq

using namespace lrq;

extern "C" int lrq_softmax_bwd(const lrq_tensors* t, const void* dp, int64_t lddp, void* ds, int64_t ldds,
                               void* stream) {
  int st = validate_tensors(t);
  if (st) return st;
  st = validate_rows16(dp, lddp, t->hidden);
  if (st) return st;
  st = validate_rows16(ds, ldds, t->hidden);
  if (st) return st;
  if (t->rows == 0) return LRQ_OK;
  hipStream_t s = (hipStream_t)stream;
  if ((t->flags & LRQ_FLAG_HADAMARD) && t->n_outlier == 0 && (t->hidden / (8 / t->bits)) % 128 == 0) {
    LRQ_FORMATS(softmax_rot_launch, t, dp, lddp, ds, ldds, s)
  }
  if ((t->flags & LRQ_FLAG_HADAMARD) || t->n_outlier > 0) {
    // outlier channels, and the rotated format with planes that are not whole rotation blocks:
    // decode into ds (rotation undone, side columns substituted), then the dense backward in
    // place over it; rows of exactly `hidden` elements, and ds distinct from dp (the decode
    // would overwrite dp before the backward reads it)
    if (lddp != t->hidden || ldds != t->hidden || dp == ds) return LRQ_ERR_UNSUPPORTED;
    LRQ_TRY(lrq_decode(t, ds, ldds, stream));
    return lrq_dense_softmax_bwd(ds, dp, ds, t->rows, t->hidden, stream);
  }
  LRQ_FORMATS(softmax_units, t, dp, lddp, ds, ldds, s)
}

extern "C" int lrq_dequant_gemm(const lrq_tensors* t, const void* a, int32_t n_out, void* out, int64_t ldo,
                                int32_t out_fp32, void* stream) {
  int st = validate_tensors(t);
  if (st) return st;
  if (a == nullptr || out == nullptr) return LRQ_ERR_NULL;
  if (n_out != 16 && n_out != 32) return LRQ_ERR_UNSUPPORTED;
  if (ldo < n_out) return LRQ_ERR_SHAPE;
  if (!aligned(a, 8) || !aligned(out, out_fp32 ? 4 : 2)) return LRQ_ERR_ALIGN;
  if (t->n_outlier > kSideGemmMax) return LRQ_ERR_UNSUPPORTED;
  if (t->rows == 0) return LRQ_OK;
  hipStream_t s = (hipStream_t)stream;
  const bool f32 = out_fp32 != 0;
  LRQ_FORMATS(gemm_nout, t, a, n_out, out, ldo, f32, s)
}

// The rotated format needs planes of whole rotation blocks.
static bool gemm_t_format_ok(const lrq_tensors* t) {
  return !(t->flags & LRQ_FLAG_HADAMARD) || (t->hidden / (8 / t->bits)) % 128 == 0;
}

static GemmTPlan gemm_t_plan(const lrq_tensors* t, int n_out) {
  return gemm_t_plan(t->rows, t->hidden, t->bits, t->group, t->rank, n_out, (t->flags & LRQ_FLAG_HADAMARD) != 0);
}

extern "C" int64_t lrq_dequant_gemm_t_workspace(const lrq_tensors* t, int32_t n_out) {
  int st = validate_tensors(t);
  if (st) return st;
  if (n_out != 16 && n_out != 32) return LRQ_ERR_UNSUPPORTED;
  if (!gemm_t_format_ok(t)) return LRQ_ERR_UNSUPPORTED;
  return gemm_t_plan(t, n_out).ws_bytes;
}

extern "C" int lrq_dequant_gemm_t(const lrq_tensors* t, const void* g, int64_t ldg, int32_t n_out, void* out,
                                  int64_t ldo, int32_t out_fp32, void* workspace, int64_t workspace_bytes,
                                  void* stream) {
  int st = validate_tensors(t);
  if (st) return st;
  if (g == nullptr || out == nullptr) return LRQ_ERR_NULL;
  if (n_out != 16 && n_out != 32) return LRQ_ERR_UNSUPPORTED;
  if (ldg < n_out || ldo < n_out) return LRQ_ERR_SHAPE;
  if (!aligned(g, 8) || (ldg % 4) != 0 || !aligned(out, out_fp32 ? 4 : 2)) return LRQ_ERR_ALIGN;
  if (!gemm_t_format_ok(t)) return LRQ_ERR_UNSUPPORTED;
  const GemmTPlan pl = gemm_t_plan(t, n_out);
  if (pl.ws_bytes > 0) {
    if (workspace == nullptr) return LRQ_ERR_NULL;
    if (workspace_bytes < pl.ws_bytes) return LRQ_ERR_WORKSPACE;
    if (!aligned(workspace, 16)) return LRQ_ERR_ALIGN;
  }
  hipStream_t s = (hipStream_t)stream;
  const bool f32 = out_fp32 != 0;
  float* ws = reinterpret_cast<float*>(workspace);
  LRQ_TRY([&]() -> int { LRQ_FORMATS(gemm_t_nout, t, g, ldg, n_out, out, ldo, f32, ws, pl, s) }());
  return side_gemm_t(t, g, ldg, n_out, out, ldo, f32, s);
}

extern "C" int lrq_dequant_gemm_t_noalloc(const lrq_tensors* t, const void* g, int64_t ldg, int32_t n_out, void* out,
                                          int64_t ldo, int32_t out_fp32, void* stream) {
  int st = validate_tensors(t);
  if (st) return st;
  if (g == nullptr || out == nullptr) return LRQ_ERR_NULL;
  if (n_out != 16 && n_out != 32) return LRQ_ERR_UNSUPPORTED;
  if (ldg < n_out || ldo < n_out) return LRQ_ERR_SHAPE;
  if (!aligned(g, 8) || (ldg % 4) != 0 || !aligned(out, out_fp32 ? 4 : 2)) return LRQ_ERR_ALIGN;
  if (!gemm_t_format_ok(t)) return LRQ_ERR_UNSUPPORTED;
  const GemmTPlan pl = gemm_t_plan(t, n_out);
  if (pl.ws_bytes > (int64_t)LRQ_GEMM_T_SCRATCH_BYTES) return LRQ_ERR_WORKSPACE;
  float* ws = nullptr;
  st = scratch_on_current_device(&ws);
  if (st) return st;
  hipStream_t s = (hipStream_t)stream;
  const bool f32 = out_fp32 != 0;
  LRQ_TRY([&]() -> int { LRQ_FORMATS(gemm_t_nout, t, g, ldg, n_out, out, ldo, f32, ws, pl, s) }());
  return side_gemm_t(t, g, ldg, n_out, out, ldo, f32, s);
}
