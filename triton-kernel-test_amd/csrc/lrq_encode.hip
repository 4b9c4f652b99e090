// Group-mode encode: projection L = bf16(X V), residual R = X - L V^T, per-group
// asymmetric quantisation and row-planar packing.
//
// Implementations, chosen per call by lrq_encode():
//   * k_encode_persist — one pass over X (about one workgroup per CU).  The NW waves
//     split the hidden dimension into units; each wave keeps the reconstruction operands of
//     its units (V rows) in registers for the whole kernel, and its share of the current
//     16-row block of X in registers while the next block streams in (double buffer).  The
//     projection's V^T operand is regenerated from the register-resident V operand with an
//     identity MFMA, so V is read from memory once per workgroup.  Partial L tiles go
//     through LDS; each wave sums a 1/NW slice of the tile and writes it as bf16, and every
//     wave reads back its rows of L (two barriers per row block, neither of which waits for
//     the prefetch).
//   * k_project + k_quant — two passes for other shapes (rank 32, hidden sizes without a
//     persistent instantiation); X is read twice.  k_quant alone is the whole rank-0 encode
//     (with optional outlier channels).
#include "lrq_common.h"
#include "lrq_host.h"
#include "lrq_quant.h"
#include "lrq_whtop.h"

#include <type_traits>

namespace lrq {

// -------------------------------------------------------------------------------------
// Single-pass encode.  Grid: ceil(row blocks / RBW) workgroups of NW waves (about one per
// CU); wave w owns units [w*UPW, (w+1)*UPW).  The host guarantees N == NW*UPW*G*NP and
// R == 16*RT.
// VLDS: the waves' V operands live in LDS (read right before each use) instead of registers,
// which leaves room for the double-buffered X tile.
template <int BITS, int G, int R, int NW, int UPW>
struct PersistLds {
  static constexpr int kVopPerWave = UPW * (8 / BITS) * (G / 16) * (R / 16);  // u32x2 per lane
  static constexpr size_t kVopBytes = (size_t)NW * kVopPerWave * 64 * 8;
  static constexpr size_t kPartBytes = (size_t)NW * (R / 16) * 64 * 16;  // per-wave partial L tiles
  static constexpr size_t kLBytes = (size_t)16 * R * 2;                  // reduced L tile, bf16
  static constexpr size_t kRedBytes = kPartBytes + kLBytes;
};

template <int BITS, int G, int R, int NW, int UPW, bool DB, bool VLDS, int RBW>
__global__ __launch_bounds__(NW * 64) void k_encode_persist(
    const uint16_t* __restrict__ X, int64_t ldx, int M, int N, const uint16_t* __restrict__ V,
    uint16_t* __restrict__ Lout, int64_t ldl, uint8_t* __restrict__ codes, int64_t ldc,
    uint16_t* __restrict__ qparams, int64_t ldq) {
  constexpr int NP = 8 / BITS, CPG = G / 32, RT = R / 16, E = G / 4;
  using Lds = PersistLds<BITS, G, R, NW, UPW>;
  extern __shared__ __attribute__((aligned(16))) unsigned char shm[];
  f32x4* part = reinterpret_cast<f32x4*>(shm);                              // [NW][RT][64]
  uint16_t* ltile = reinterpret_cast<uint16_t*>(shm + Lds::kPartBytes);     // [16][R]
  u32x2* vlds = reinterpret_cast<u32x2*>(shm + Lds::kRedBytes);             // [NW][kVopPerWave][64]
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int j = lane & 15, g = lane >> 4;
  const int nrb = (M + 15) / 16;

  u32x2 vreg[VLDS ? 1 : UPW][NP][G / 16][RT];
#pragma unroll
  for (int uu = 0; uu < UPW; ++uu)
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      u32x2 tmp[G / 16][RT];
      load_vops<G, R>(V, unit_base(p, w * UPW + uu, N, NP, G), j, g, tmp);
#pragma unroll
      for (int q = 0; q < G / 16; ++q)
#pragma unroll
        for (int t = 0; t < RT; ++t) {
          if constexpr (VLDS)
            vlds[(w * Lds::kVopPerWave + ((uu * NP + p) * (G / 16) + q) * RT + t) * 64 + lane] = tmp[q][t];
          else
            vreg[uu][p][q][t] = tmp[q][t];
        }
    }
  // V operands of unit uu, plane p (from registers, or LDS where this wave wrote them)
  auto vops = [&](int uu, int p, u32x2 (&out)[G / 16][RT]) {
#pragma unroll
    for (int q = 0; q < G / 16; ++q)
#pragma unroll
      for (int t = 0; t < RT; ++t) {
        if constexpr (VLDS)
          out[q][t] = vlds[(w * Lds::kVopPerWave + ((uu * NP + p) * (G / 16) + q) * RT + t) * 64 + lane];
        else
          out[q][t] = vreg[VLDS ? 0 : uu][p][q][t];
      }
  };
  const u32x2 ident = identity_bop(j, g);

  // Load the lane's share of row block rb (when !valid every lane reads X[0..15] instead).
  auto load = [&](u32x4 (&x)[UPW][NP][CPG], int rb, bool valid) {
    const int row = min(rb * 16 + j, M - 1);
    const uint16_t* xr = X + (int64_t)row * ldx + E * g;
#pragma unroll
    for (int uu = 0; uu < UPW; ++uu)
#pragma unroll
      for (int p = 0; p < NP; ++p)
#pragma unroll
        for (int k = 0; k < CPG; ++k) {
          const uint16_t* a = xr + unit_base(p, w * UPW + uu, N, NP, G) + 8 * k;
          x[uu][p][k] = ld16_stream(valid ? a : X);
        }
    // keep the prefetch where it is issued (the scheduler would sink it next to its use,
    // behind the previous block's stores)
    __builtin_amdgcn_sched_barrier(0);
  };

  // The L tile of a row block is RT*256 fp32 sums over NW partials; wave w reduces floats
  // [w*F, (w+1)*F): lane l adds partials (l/F)*PPL .. +PPL-1 of float l%F, and the S lanes
  // holding the same float combine with xor-shuffles.
  constexpr int F = RT * 256 / NW, S = 64 / F, PPL = NW / S;
  static_assert(F >= 1 && F <= 64 && 64 % F == 0 && NW % S == 0, "L reduction split");
  const float* partf = reinterpret_cast<const float*>(part);

  auto process = [&](const u32x4 (&x)[UPW][NP][CPG], int rb) {
    const int row = min(rb * 16 + j, M - 1);  // rows past the end repeat the last row (see load)
    // two accumulator chains (even / odd unit-plane) to halve the dependent MFMA sequence
    f32x4 acc[2][RT];
#pragma unroll
    for (int t = 0; t < RT; ++t) acc[0][t] = acc[1][t] = zero4();
#pragma unroll
    for (int uu = 0; uu < UPW; ++uu)
#pragma unroll
      for (int p = 0; p < NP; ++p) {
        u32x2 v[G / 16][RT];
        vops(uu, p, v);
        project_unit<G, R>(v, x[uu][p], ident, acc[(uu * NP + p) & 1]);
      }
#pragma unroll
    for (int t = 0; t < RT; ++t) {
      f32x4 a = acc[0][t];
      a[0] += acc[1][t][0];
      a[1] += acc[1][t][1];
      a[2] += acc[1][t][2];
      a[3] += acc[1][t][3];
      part[(w * RT + t) * 64 + lane] = a;
    }
    lds_barrier();
    {
      const int f = lane % F, pg = lane / F;
      const int fi = w * F + f;                          // float of the tile: (t, source lane, v)
      const int t = fi >> 8, src = (fi >> 2) & 63, v = fi & 3;
      float sum = 0.f;
#pragma unroll
      for (int i = 0; i < PPL; ++i) sum += partf[(((pg * PPL + i) * RT + t) * 64 + src) * 4 + v];
#pragma unroll
      for (int m = F; m < 64; m <<= 1) sum += __shfl_xor(sum, m);
      // source lane (j', g') of partial tile t holds L[row j'][16t + 4g' + v]
      if (pg == 0) ltile[(src & 15) * R + 16 * t + 4 * (src >> 4) + v] = (uint16_t)pack_bf16x2(sum, 0.f);
    }
    lds_barrier();
    u32x2 lop[RT], lopn[RT];
#pragma unroll
    for (int t = 0; t < RT; ++t) {
      lop[t] = *reinterpret_cast<const u32x2*>(ltile + j * R + 16 * t + 4 * g);
      lopn[t] = neg_bf16x4(lop[t]);
      // wave 0 stores the tile (rows past the end rewrite the last row's L)
      st8_pred(Lout + (int64_t)rb * 16 * ldl, (uint32_t)(16 * ldl * 2),
               (uint32_t)(((row - rb * 16) * ldl + 16 * t + 4 * g) * 2), lop[t], w == 0);
    }
    uint8_t* crow = codes + (int64_t)rb * 16 * ldc + (uint32_t)(row - rb * 16) * (uint32_t)ldc;
    uint16_t* qrow = qparams + (int64_t)row * ldq;
#pragma unroll
    for (int uu = 0; uu < UPW; ++uu) {
      u32x2 v[NP][G / 16][RT];
#pragma unroll
      for (int p = 0; p < NP; ++p) vops(uu, p, v[p]);
      quant_unit<BITS, G, R>(x[uu], v, lopn, nullptr, w * UPW + uu, N, g, crow, qrow);
    }
    __builtin_amdgcn_sched_barrier(0);  // keep row blocks from interleaving (register pressure)
  };

  // RBW row blocks per workgroup, straight-line: block b+1 is requested before block b is
  // processed (two register buffers, indices fixed after unrolling).  Blocks past the end
  // (tail workgroup only) repeat the last block and rewrite the same bytes.
  const int rb0 = blockIdx.x * RBW;
  u32x4 xs[DB ? 2 : 1][UPW][NP][CPG];
  load(xs[0], min(rb0, nrb - 1), true);
#pragma unroll
  for (int b = 0; b < RBW; ++b) {
    if constexpr (DB) {
      if (b + 1 < RBW) load(xs[(b + 1) & 1], min(rb0 + b + 1, nrb - 1), true);
      process(xs[b & 1], min(rb0 + b, nrb - 1));
    } else {
      if (b > 0) load(xs[0], min(rb0 + b, nrb - 1), true);
      process(xs[0], min(rb0 + b, nrb - 1));
    }
  }
}

// -------------------------------------------------------------------------------------
// Row-staged single-pass encode (about one workgroup per CU, NW waves of UPW units each).
//
// On MI355X a CU has a small budget of loads in flight (about its L1 size) and serves its
// memory instructions in issue order; loads in the MFMA layout (16 rows x 4 x 16 B per
// instruction) reach far less bandwidth than contiguous ones.  Here each wave streams its own
// slice of the next row block (16 rows x NP pieces of UPW*G*2 contiguous bytes) into a private
// LDS region, in NR rounds interleaved with the current block's work, and reads it back in the
// MFMA layout.  The region is private, so the only barrier per block is the one that publishes
// the projection partials (double-buffered; every lane sums the NW partials of its own lane
// position in a fixed order, so L is deterministic).  V operands stay in registers for the
// whole kernel.  Rows past the end repeat the last row (no predicated stores).
template <int BITS, int G, int R, int NW, int UPW>
struct RowsEnc {
  static constexpr int NP = 8 / BITS, RT = R / 16;
  static constexpr int PIECE = UPW * G * 2;         // bytes of one (row, plane) piece of a slice
  static constexpr int PITCH = NP * PIECE + 16;      // LDS row pitch of a region (bank spread)
  static constexpr int REGION = 16 * PITCH;          // bytes per wave
  static constexpr int PPL = 1024 / PIECE;           // pieces per 1 KB load instruction
  static constexpr int LPL = 64 / PPL;               // lanes per piece
  static constexpr int NLD = 16 * NP / PPL;          // load instructions per wave and block
  static constexpr int NR = 4, RL = NLD / NR;        // rounds per block, loads per round
  static constexpr int PART = NW * RT * 64 * 16;     // one partial slot
  static constexpr size_t LDS = (size_t)NW * REGION + 2 * (size_t)PART;
  static_assert(1024 % PIECE == 0 && NLD % NR == 0 && NR == 4, "slice pieces per load; the round schedule is written for 4");
  static_assert(LDS <= 160 * 1024, "LDS budget");
};

// Direct-to-LDS slices (RowsEnc::PPL == NP): the next block's 16 row loads are issued in
// pieces at points 0 (after the current slice is read), 1 (after the partial sums) and 2 + u
// (after unit u is quantised); n[pt] loads at point pt.
template <int UPW>
struct DmaSched;
template <>
struct DmaSched<4> {
  static constexpr int n[6] = {4, 8, 0, 4, 0, 0};
};
template <>
struct DmaSched<2> {
  static constexpr int n[4] = {4, 8, 0, 4};
};
// loads issued before point pt
template <int UPW>
constexpr int dma_begin(int pt) {
  int s = 0;
  for (int i = 0; i < pt; ++i) s += DmaSched<UPW>::n[i];
  return s;
}
// units quantised after the last point that issues loads
template <int UPW>
constexpr int dma_units_after() {
  int last = 0;
  for (int i = 0; i < UPW + 2; ++i)
    if (DmaSched<UPW>::n[i] > 0) last = i;
  return last < 2 ? UPW : UPW - 1 - (last - 2);
}

// OUTL: outlier channels.  The V operand rows of outlier columns are zeroed once, so the
// projection is that of Y with those columns zeroed (the same products and sums) and their
// residuals are zeroed before the group statistics; their bf16 values go to the fp16 side
// columns from the slice in LDS.  LDS: Re::LDS + N/32 mask words + N slot entries.
template <int BITS, int G, int R, int NW, int UPW, bool OUTL>
__global__ __launch_bounds__(NW * 64) void k_encode_rows(
    const uint16_t* __restrict__ X, int64_t ldx, int M, int N, const uint16_t* __restrict__ V,
    uint16_t* __restrict__ Lout, int64_t ldl, uint8_t* __restrict__ codes, int64_t ldc,
    uint16_t* __restrict__ qparams, int64_t ldq, int RBW, const int32_t* __restrict__ oidx, int nout,
    uint16_t* __restrict__ side, int64_t ldside) {
  using Re = RowsEnc<BITS, G, R, NW, UPW>;
  constexpr int NP = Re::NP, CPG = G / 32, RT = Re::RT, E = G / 4;
  static_assert(NP == 2 && (UPW == 2 || UPW == 4), "the qparams gather below is written for 2 planes x 2 or 4 units");
  extern __shared__ __attribute__((aligned(16))) unsigned char shm[];
  const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
  const int j = lane & 15, g = lane >> 4;
  unsigned char* region = shm + (size_t)w * Re::REGION;
  f32x4* part = reinterpret_cast<f32x4*>(shm + (size_t)NW * Re::REGION);  // [2][NW][RT][64]
  const int nrb = (M + 15) / 16;
  const int rb0 = blockIdx.x * RBW;
  if (rb0 >= nrb) return;  // whole workgroup (no barrier reached)
  const int nblk = min(RBW, nrb - rb0);
  const int ub = w * UPW;  // first unit of this wave
  uint32_t* colmask = reinterpret_cast<uint32_t*>(shm + Re::LDS);  // OUTL: N/32 words
  int16_t* oslot = reinterpret_cast<int16_t*>(colmask + N / 32);   // OUTL: N entries
  if constexpr (OUTL) {
    for (int i = threadIdx.x; i < N / 32; i += NW * 64) colmask[i] = 0u;
    for (int i = threadIdx.x; i < N; i += NW * 64) oslot[i] = -1;
    __syncthreads();
    for (int k = threadIdx.x; k < nout; k += NW * 64) {
      const int c = oidx[k];
      if (c >= 0 && c < N) {
        atomicOr(&colmask[c >> 5], 1u << (c & 31));
        oslot[c] = (int16_t)k;
      }
    }
    __syncthreads();
  }
  // zero the V operand rows of outlier columns (lane (j, g) of operand q holds V row
  // vrow_res(base, j, q))
  auto mask_vops = [&](u32x2 (&vo)[UPW][NP][G / 16][RT]) {
    if constexpr (OUTL) {
#pragma unroll
      for (int uu = 0; uu < UPW; ++uu)
#pragma unroll
        for (int p = 0; p < NP; ++p)
#pragma unroll
          for (int q = 0; q < G / 16; ++q) {
            const int c = vrow_res<G>(unit_base(p, ub + uu, N, NP, G), j, q);
            const bool z = (colmask[c >> 5] >> (c & 31)) & 1u;
#pragma unroll
            for (int t = 0; t < RT; ++t) vo[uu][p][q][t] = z ? u32x2{0u, 0u} : vo[uu][p][q][t];
          }
    }
  };
  // side columns of the wave's units, read from the slice in the region (lanes of quarter 0
  // store row j; rows past the end repeat the last row)
  auto side_store = [&](int rb, int row) {
    if constexpr (OUTL) {
      const __amdgpu_buffer_rsrc_t rs =
          uniform_rsrc(side + (int64_t)rb * 16 * ldside, (uint32_t)(16 * ldside * 2));
#pragma unroll
      for (int p = 0; p < NP; ++p) {
        const int cb = unit_base(p, ub, N, NP, G);  // the wave's UPW*G contiguous columns of plane p
#pragma unroll 1
        for (int wd = 0; wd < UPW * G / 32; ++wd) {
          uint32_t bits = __builtin_amdgcn_readfirstlane(colmask[(cb >> 5) + wd]);
          while (bits != 0u) {
            const int e = __builtin_ctz(bits);
            bits &= bits - 1u;
            const int cl = 32 * wd + e;  // column within the wave's range
            const int k = oslot[cb + cl];
            const uint32_t v = *reinterpret_cast<const uint16_t*>(region + j * Re::PITCH + p * Re::PIECE + cl * 2);
            const uint16_t h = (uint16_t)f16_bits(__uint_as_float(v << 16));
            __builtin_amdgcn_raw_buffer_store_b16(h, rs, g == 0 ? (uint32_t)(((row - rb * 16) * ldside + k) * 2) : 0x7ffffff0u,
                                                  0, 0);
          }
        }
      }
    }
  };

  // With one row per load instruction (RPL == 1) a load's 1 KB lands contiguously in the
  // region, so it goes straight from HBM to LDS (no staging registers); the registers saved
  // hold the projection's V^T operands for the whole kernel.
  constexpr bool DMA = Re::PPL == NP;
  u32x2 vop[UPW][NP][G / 16][RT];
  u32x4 vt[DMA ? UPW : 1][NP][CPG][RT];
  const u32x2 ident = identity_bop(j, g);

  // Load instruction i of block rb covers rows RPL*i .. RPL*i + RPL-1 of the block (RPL = PPL/NP
  // rows), every plane: lane l carries 16 bytes of piece i*PPL + l/LPL (row RPL*i + (l/LPL)/NP,
  // plane (l/LPL)%NP) at byte (l % LPL) * 16 of the wave's piece.  The first row's address is
  // wave-uniform (scalar); the lane part is a fixed 32-bit offset.  Rows past the end are
  // clamped to the last row, which only the last block can reach.
  static_assert(Re::PPL % NP == 0, "whole rows per load instruction");
  constexpr int RPL = Re::PPL / NP;
  const int lpc = lane / Re::LPL, loff = (lane % Re::LPL) * 16;
  const int lrow = lpc / NP;  // row within the instruction's RPL rows
  const uint32_t xlane = (uint32_t)unit_base(lpc % NP, ub, N, NP, G) * 2u + (uint32_t)loff;
  auto gaddr = [&](int rb, int i) {
    const int64_t r0 = rb * 16 + RPL * i;
    if (r0 + RPL <= M)  // every row of the instruction present (all but possibly the last block)
      return reinterpret_cast<const unsigned char*>(X + r0 * ldx) + (uint32_t)(lrow * ldx * 2) + xlane;
    const int64_t row = min(r0 + lrow, (int64_t)M - 1);
    return reinterpret_cast<const unsigned char*>(X + row * ldx) + xlane;
  };
  auto laddr = [&](int i) {
    return region + (RPL * i + lrow) * Re::PITCH + (lpc % NP) * Re::PIECE + loff;
  };
  u32x4 pf[DMA ? 1 : 2][Re::RL];
  auto issue = [&](int buf, int rb, int round) {
#pragma unroll
    for (int i = 0; i < Re::RL; ++i) {
      if constexpr (DMA)
        ld16_to_lds(gaddr(rb, round * Re::RL + i), region + (round * Re::RL + i) * Re::PITCH);
      else
        pf[buf][i] = ld16_stream(gaddr(rb, round * Re::RL + i));
    }
  };
  // DMA: the loads of schedule point pt (rows dma_begin(pt) .. dma_begin(pt + 1) - 1)
  auto issue_pt = [&](auto pt_tag, int rb) {
    constexpr int pt = decltype(pt_tag)::value;
    if constexpr (DMA)
      static_for<dma_begin<UPW>(pt), dma_begin<UPW>(pt + 1)>(
          [&](auto i) { ld16_to_lds(gaddr(rb, i), region + (int)i * Re::PITCH); });
  };
  auto land = [&](int buf, int round) {
    if constexpr (!DMA) {
#pragma unroll
      for (int i = 0; i < Re::RL; ++i) *reinterpret_cast<u32x4*>(laddr(round * Re::RL + i)) = pf[buf][i];
    }
  };

  // Prologue: block rb0 into the region, two rounds in flight.  The first two rounds are
  // requested before the V operands (L2-resident after the first workgroups), so HBM is busy
  // from the start.  V arrives as whole 1 KB pieces (the wave's V rows are NP contiguous ranges
  // of UPW*G rows), passes through the region, and is read back in the operand layout before
  // the region receives block rb0.
  if constexpr (DMA) {
    // The whole of block rb0 first (HBM), then the V operands (L2-resident after the first
    // workgroups) in the residual layout, transposed once for the projection: the memory
    // pipeline serves a wave's requests in order, so X's requests leave before V's.
    const int rb = min(rb0, nrb - 1);
#pragma unroll
    for (int rd = 0; rd < Re::NR; ++rd) issue(0, rb, rd);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int uu = 0; uu < UPW; ++uu)
#pragma unroll
      for (int p = 0; p < NP; ++p) load_vops<G, R>(V, unit_base(p, ub + uu, N, NP, G), j, g, vop[uu][p]);
    __builtin_amdgcn_sched_barrier(0);
    mask_vops(vop);
#pragma unroll
    for (int uu = 0; uu < UPW; ++uu)
#pragma unroll
      for (int p = 0; p < NP; ++p) transpose_vops<G, R>(vop[uu][p], ident, vt[uu][p]);
  } else {
    const int rb = min(rb0, nrb - 1);
    issue(0, rb, 0);
    issue(1, rb, 1);
    __builtin_amdgcn_sched_barrier(0);
    constexpr int VB = UPW * G * R * 2;  // bytes of the wave's V rows in one plane
    constexpr int VLD = NP * VB / 1024;   // 1 KB loads
    static_assert(VB % 1024 == 0 && NP * VB <= Re::REGION, "V staging through the region");
    u32x4 vraw[VLD];
#pragma unroll
    for (int i = 0; i < VLD; ++i) {
      const int p = i / (VB / 1024);
      vraw[i] = ld16(reinterpret_cast<const unsigned char*>(V + (int64_t)unit_base(p, ub, N, NP, G) * R) +
                     (i % (VB / 1024)) * 1024 + lane * 16);
    }
#pragma unroll
    for (int i = 0; i < VLD; ++i) *reinterpret_cast<u32x4*>(region + i * 1024 + lane * 16) = vraw[i];
#pragma unroll
    for (int uu = 0; uu < UPW; ++uu)
#pragma unroll
      for (int p = 0; p < NP; ++p)
#pragma unroll
        for (int q = 0; q < G / 16; ++q)
#pragma unroll
          for (int t = 0; t < RT; ++t) {
            const int vr = uu * G + vrow_res<G>(0, j, q);  // V row within the plane's range
            vop[uu][p][q][t] = *reinterpret_cast<const u32x2*>(region + p * VB + vr * R * 2 + 32 * t + 8 * g);
          }
    mask_vops(vop);
    // the region is rewritten below: every read above must have returned
    __builtin_amdgcn_s_waitcnt(0xc07f);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int rd = 0; rd < Re::NR; ++rd) {
      land(rd & 1, rd);
      if (rd + 2 < Re::NR) issue(rd & 1, rb, rd + 2);
    }
  }

  // One row block; NEXT: stream the next block's slice into the region meanwhile.  The block
  // loop is not unrolled (unrolled, the compiler's schedule across blocks spills registers).
  auto block = [&](auto next_tag, int b) {
    constexpr bool next = decltype(next_tag)::value;
    const int rb = __builtin_amdgcn_readfirstlane(min(rb0 + b, nrb - 1));  // wave-uniform
    const int row = min(rb * 16 + j, M - 1);
    const int rbn = __builtin_amdgcn_readfirstlane(min(rb0 + b + 1, nrb - 1));
    if constexpr (DMA) {
      // Wait until the slice's loads have written the region.  vmcnt retires in issue order
      // on gfx9 (loads and stores alike); after the last of a block's loads this wave issues
      // exactly kAfter stores (the codes of the units quantised after it, the qparams and L
      // rows), which need not complete here.  Block 0's loads are the prologue's last memory
      // operations.
      static_assert(dma_begin<UPW>(UPW + 2) == Re::NLD, "the schedule issues every load of a block once");
      constexpr int kAfter = dma_units_after<UPW>() * quant_core_stores<G>() + 1 + RT;
      static_assert(kAfter < 16, "vmcnt immediate");
      if (b == 0)
        __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0)
      else
        __builtin_amdgcn_s_waitcnt(0x0f70 | kAfter);
      __builtin_amdgcn_sched_barrier(0);
    }
    // this block's slice, MFMA layout (lane (j, g): row j, columns E*g .. of each unit-plane)
    u32x4 x[UPW][NP][CPG];
#pragma unroll
    for (int uu = 0; uu < UPW; ++uu)
#pragma unroll
      for (int p = 0; p < NP; ++p)
#pragma unroll
        for (int k = 0; k < CPG; ++k)
          x[uu][p][k] = *reinterpret_cast<const u32x4*>(region + j * Re::PITCH + p * Re::PIECE + (uu * G + E * g + 8 * k) * 2);
    side_store(rb, row);
    if constexpr (DMA) {
      // the region may be overwritten once every read of the slice has returned
      __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
      __builtin_amdgcn_sched_barrier(0);
    }
    if (next) {
      if constexpr (DMA)
        issue_pt(std::integral_constant<int, 0>{}, rbn);
      else
        issue(0, rbn, 0);
    }
    __builtin_amdgcn_sched_barrier(0);

    f32x4 acc[2][RT];
#pragma unroll
    for (int t = 0; t < RT; ++t) acc[0][t] = acc[1][t] = zero4();
#pragma unroll
    for (int uu = 0; uu < UPW; ++uu)
#pragma unroll
      for (int p = 0; p < NP; ++p) {
        if constexpr (DMA)
          project_unit_vt<G, R>(vt[uu][p], x[uu][p], acc[(uu * NP + p) & 1]);
        else
          project_unit<G, R>(vop[uu][p], x[uu][p], ident, acc[(uu * NP + p) & 1]);
      }
    f32x4* slot = part + (size_t)(b & 1) * NW * RT * 64;
#pragma unroll
    for (int t = 0; t < RT; ++t) {
      f32x4 a = acc[0][t];
      a[0] += acc[1][t][0];
      a[1] += acc[1][t][1];
      a[2] += acc[1][t][2];
      a[3] += acc[1][t][3];
      slot[(w * RT + t) * 64 + lane] = a;
    }
    lds_barrier();
    u32x2 lop[RT], lopn[RT];
#pragma unroll
    for (int t = 0; t < RT; ++t) {
      f32x4 s = slot[t * 64 + lane];
#pragma unroll
      for (int w2 = 1; w2 < NW; ++w2) {
        const f32x4 o = slot[(w2 * RT + t) * 64 + lane];
        s[0] += o[0];
        s[1] += o[1];
        s[2] += o[2];
        s[3] += o[3];
      }
      // lane (j, g) holds L[row j][16t + 4g + v]
      lop[t] = u32x2{pack_bf16x2(s[0], s[1]), pack_bf16x2(s[2], s[3])};
      lopn[t] = neg_bf16x4(lop[t]);
    }
    // the region's rows of the next block arrive round by round between the quantised units
    // (at most two rounds in flight: round 0 overlaps the projection, 1 and 2 the first two
    // units, 3 the last two)
    if (next) {
      if constexpr (DMA) {
        issue_pt(std::integral_constant<int, 1>{}, rbn);
      } else {
        land(0, 0);
        issue(1, rbn, 1);
        issue(0, rbn, 2);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    uint8_t* crow = codes + (int64_t)rb * 16 * ldc + (uint32_t)(row - rb * 16) * (uint32_t)ldc;
    uint32_t qp[UPW];
#pragma unroll
    for (int uu = 0; uu < UPW; ++uu) {
      if constexpr (OUTL)
        qp[uu] = quant_unit_core<BITS, G, R>(x[uu], vop[uu], lopn, colmask, ub + uu, N, g, crow);
      else
        qp[uu] = quant_unit_regs<BITS, G, R>(x[uu], vop[uu], lopn, ub + uu, g, crow);
      if constexpr (DMA) {
        if (next)
          static_for<0, UPW>([&](auto u) {
            if (uu == u && DmaSched<UPW>::n[2 + u] > 0) {
              __builtin_amdgcn_sched_barrier(0);
              issue_pt(std::integral_constant<int, 2 + u>{}, rbn);
              __builtin_amdgcn_sched_barrier(0);
            }
          });
      } else if (uu == 1 && next) {
        __builtin_amdgcn_sched_barrier(0);
        land(1, 1);
        issue(1, rbn, 3);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    // qparams of the wave's units as 16-byte stores per row: lanes 0..31 hold the plane-0
    // pairs, lanes 32..63 the plane-1 pairs, and the row's memory order is (unit, plane).
    // Four units: two half-swaps leave units 0-1 in the low lanes and units 2-3 in the high
    // lanes.  Two units: the half-swaps pair each plane-0 value with its plane-1 partner in the
    // low lanes, which store.
    {
      float a, bq, c, d;
      if constexpr (UPW == 4) {
        a = __uint_as_float(qp[0]), bq = __uint_as_float(qp[2]);
        c = __uint_as_float(qp[1]), d = __uint_as_float(qp[3]);
      } else {
        a = bq = __uint_as_float(qp[0]);
        c = d = __uint_as_float(qp[1]);
      }
      swap32(a, bq);
      swap32(c, d);
      const u32x4 v = u32x4{__float_as_uint(a), __float_as_uint(bq), __float_as_uint(c), __float_as_uint(d)};
      const bool keep = UPW == 4 ? (g & 1) == 0 : g == 0;
      st16_pred(qparams + (int64_t)rb * 16 * ldq, (uint32_t)(16 * ldq * 2),
                (uint32_t)(((row - rb * 16) * ldq + ub * NP * 2) * 2 + (g >> 1) * 16), v, keep);
    }
#pragma unroll
    for (int t = 0; t < RT; ++t)
      st8_pred(Lout + (int64_t)rb * 16 * ldl, (uint32_t)(16 * ldl * 2),
               (uint32_t)(((row - rb * 16) * ldl + 16 * t + 4 * g) * 2), lop[t], w == 0);
    if (next) {
      __builtin_amdgcn_sched_barrier(0);
      land(0, 2);
      land(1, 3);
    }
    __builtin_amdgcn_sched_barrier(0);
  };
#pragma unroll 1
  for (int b = 0; b < nblk - 1; ++b) block(std::true_type{}, b);
  block(std::false_type{}, nblk - 1);
}

// -------------------------------------------------------------------------------------
// Tile-staged single-pass encode for rows too wide for per-wave regions (int4/g64, NW*UPW
// units of 128 columns; 40 units = 5120 columns fill the 160 KB of LDS with one 16-row block).
//
// The block lives in LDS as N/128 tiles of 16 rows x 128 columns (4 KB): tile t holds
// columns 128t .. 128t+127, its row r at byte 256r, and the row's 16-byte chunk c (columns
// 8c .. 8c+7) at position c ^ r, so that the 16 lanes of a column quarter (rows 0..15) read
// 16 different bank groups.  A direct load (1 KB) fills 4 rows of one tile: lane l writes
// position l % 16 of row 4i + l / 16 and reads that row's chunk (l % 16) ^ row from HBM, so the
// permutation costs nothing.  Wave w loads (and, with ROT, rotates in place: WHT-128 per tile
// row, the oracle's summation order) its tiles T_i = w + NW*i, i < UPW.
//
// A CU keeps about 32 KB of loads in flight and a wave that issues more waits at the issue,
// so the next block's tiles are requested one per wave at a time (4 KB, 32 KB per CU)
// between the current block's phases, and each is rotated as soon as it has landed, between
// the current block's units:
//   [top: T_4 of this block landed, rotated] barrier; read the units' columns (MFMA layout);
//   barrier; T_0 | projection | T_1 | partials into the first KB of T_4 (this wave's slot),
//   barrier, L summed in a fixed order, barrier | T_2 | unit 0 | T_3 | unit 1 | unit 2 |
//   rotate T_0 | T_4 | unit 3 | rotate T_1 | unit 4, L store | rotate T_2, T_3.
// (A rotation needs about 50 registers; by unit 2 the first units' columns are dead.)
// Waits are counted vmcnt (memory operations retire in issue order): the number of this
// wave's memory operations issued after the tile's last load.
// Unit u of plane p is half u % 2 of tile p*NT/2 + u/2.  V operands stay in registers; the
// projection's V^T operands are regenerated each block with identity MFMAs.  Rows past the
// end repeat the last row (no predicated stores).
template <int UPW, bool ROT>
struct TilesEnc {
  static constexpr int NW = 8, NT = NW * UPW, TILE = 16 * 256;
  static constexpr size_t LDS = (size_t)NT * TILE;
  static_assert(NT % 2 == 0 && LDS <= 160 * 1024, "tiles of both planes; LDS budget");
};

template <int UPW, bool ROT>
__global__ __launch_bounds__(512) void k_encode_tiles(const uint16_t* __restrict__ X, int64_t ldx, int M, int N,
                                                      const uint16_t* __restrict__ V, uint16_t* __restrict__ Lout,
                                                      int64_t ldl, uint8_t* __restrict__ codes, int64_t ldc,
                                                      uint16_t* __restrict__ qparams, int64_t ldq, int RBW) {
  using Te = TilesEnc<UPW, ROT>;
  constexpr int BITS = 4, G = 64, R = 16, NP = 2, CPG = 2, NW = Te::NW, NT = Te::NT, TILE = Te::TILE;
  static_assert(UPW == 5, "the load / rotation schedule below is written for five tiles per wave");
  extern __shared__ __attribute__((aligned(16))) unsigned char shm[];
  const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int j = lane & 15, g = lane >> 4;
  const int nrb = (M + 15) / 16;
  const int rb0 = blockIdx.x * RBW;
  if (rb0 >= nrb) return;  // whole workgroup (no barrier reached)
  const int nblk = min(RBW, nrb - rb0);
  const int ub = w * UPW;

  // tile i of this wave: rows 4k .. 4k+3 per load; lane l covers row 4k + l/16, chunk
  // (l % 16) ^ row, landing at position l % 16 (rows past the end clamp to the last row).  The
  // address is the block's first row (wave-uniform) plus a 32-bit lane offset.
  const int lr = lane >> 4, lq = lane & 15;
  const uint32_t ldx2 = (uint32_t)ldx * 2u;
  auto tile_ptr = [&](int i) { return shm + (size_t)(w + NW * i) * TILE; };
  constexpr int kTileLoads = 4;  // load instructions per tile (4 rows each)
  auto issue_tile = [&](int rb, int i) {
    const int t = w + NW * i;
    const int lim = M - 1 - rb * 16;  // last row of the block that exists (>= 0)
    const unsigned char* base = reinterpret_cast<const unsigned char*>(X + (int64_t)rb * 16 * ldx) + 256 * t;
#pragma unroll
    for (int k = 0; k < kTileLoads; ++k) {
      const int r = 4 * k + lr;
      ld16_to_lds(base + ((uint32_t)min(r, lim) * ldx2 + 16u * (uint32_t)(lq ^ r)), tile_ptr(i) + 1024 * k);
    }
    __builtin_amdgcn_sched_barrier(0);
  };
  // wait until tile i's loads have landed (n memory operations of this wave issued after them),
  // then rotate it in place (without ROT only the wait for the block's last tile, at the top)
  auto rotate_tile = [&](int i, auto n_tag, bool top = false) {
    if (ROT || top) {
      __builtin_amdgcn_s_waitcnt(vmcnt_imm(decltype(n_tag)::value));
      __builtin_amdgcn_sched_barrier(0);
    }
    if constexpr (ROT) {
      // the sign operands, formed per use from this lane's two dwords: the empty asm hides that
      // they are loop-invariant, so they do not stay live across the quantisation (whose peak
      // is within a few registers of the budget)
      int jj = j;
      asm volatile("" : "+v"(jj));
      u32x4 op[2][2];
      wht_operands_from_pair(wht_sign_dword(jj, g, 0, false, 0), wht_sign_dword(jj, g, 0, false, 1), op);
      wht128_lds_swz(tile_ptr(i) + 256 * j, g, j, op);
    }
    __builtin_amdgcn_sched_barrier(0);
  };
  // Memory operations of this wave issued after each tile's loads, up to its rotation, from the
  // block's schedule below (T_i = the next block's tile i, U_u = unit u's stores, Ls = the L row
  // store): T_0 T_1 T_2 U_0 T_3 U_1 U_2 [rotate T_0] T_4 U_3 [rotate T_1] U_4 Ls [rotate T_2,
  // T_3] ... [rotate T_4 at the next block's top].  Any change to the schedule or to the stores
  // a unit issues changes these counts with it.
  constexpr int TL = kTileLoads, US = quant_unit_stores<G>(), LS = 1;
  using C_T0 = std::integral_constant<int, 2 * TL + US + TL + 2 * US>;
  using C_T1 = std::integral_constant<int, TL + US + TL + 2 * US + TL + US>;
  using C_T2 = std::integral_constant<int, US + TL + 2 * US + TL + 2 * US + LS>;
  using C_T3 = std::integral_constant<int, 2 * US + TL + 2 * US + LS>;
  using C_T4 = std::integral_constant<int, 2 * US + LS>;
  static_assert(C_T1::value < 64 && C_T2::value < 64, "vmcnt immediate (6 bits)");

  // Prologue: block rb0 (HBM) first, then the V operands (L2-resident after the first
  // workgroups).
#pragma unroll
  for (int i = 0; i < UPW; ++i) issue_tile(rb0, i);
  u32x2 vop[UPW][NP][G / 16][1];
#pragma unroll
  for (int uu = 0; uu < UPW; ++uu)
#pragma unroll
    for (int p = 0; p < NP; ++p) load_vops<G, R>(V, unit_base(p, ub + uu, N, NP, G), j, g, vop[uu][p]);
  f32x4* slot_own = reinterpret_cast<f32x4*>(tile_ptr(UPW - 1));  // first KB of T_4
  __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
  __builtin_amdgcn_sched_barrier(0);
  if constexpr (ROT) {
#pragma unroll
    for (int i = 0; i < UPW - 1; ++i) rotate_tile(i, std::integral_constant<int, 0>{});
  }

  auto block = [&](auto next_tag, int b) {
    constexpr bool next = decltype(next_tag)::value;
    const int rb = __builtin_amdgcn_readfirstlane(rb0 + b);
    const int row = min(rb * 16 + j, M - 1);
    // T_4 of this block: units 3, 4 and the L store of the previous block after it (none after
    // the prologue)
    if (b == 0)
      rotate_tile(UPW - 1, std::integral_constant<int, 0>{}, true);
    else
      rotate_tile(UPW - 1, C_T4{}, true);
    lds_barrier();  // every tile landed and rotated
    u32x4 x[UPW][NP][CPG];
#pragma unroll
    for (int uu = 0; uu < UPW; ++uu)
#pragma unroll
      for (int p = 0; p < NP; ++p) {
        const int u = ub + uu;
        const unsigned char* tr = shm + (size_t)(p * (NT / 2) + u / 2) * TILE + 256 * j;
#pragma unroll
        for (int k = 0; k < CPG; ++k) x[uu][p][k] = *reinterpret_cast<const u32x4*>(tr + 16 * ((8 * (u & 1) + 2 * g + k) ^ j));
      }
    lds_barrier();  // every wave's reads of the block returned: the tiles may be refilled
    if (next) issue_tile(rb + 1, 0);

    f32x4 acc[2][1];
    acc[0][0] = acc[1][0] = zero4();
    {
      int jj = j;  // (as for the rotation's operands)
      asm volatile("" : "+v"(jj));
      const u32x2 ident = identity_bop(jj, g);
#pragma unroll
      for (int uu = 0; uu < UPW; ++uu)
#pragma unroll
        for (int p = 0; p < NP; ++p) project_unit<G, R>(vop[uu][p], x[uu][p], ident, acc[(uu * NP + p) & 1]);
    }
    __builtin_amdgcn_sched_barrier(0);
    if (next) issue_tile(rb + 1, 1);
    {
      f32x4 a = acc[0][0];
      a[0] += acc[1][0][0];
      a[1] += acc[1][0][1];
      a[2] += acc[1][0][2];
      a[3] += acc[1][0][3];
      slot_own[lane] = a;
    }
    lds_barrier();
    u32x2 lop[1], lopn[1];
    {
      // the eight waves' partials of this lane position, in wave order
      f32x4 sacc = zero4();
#pragma unroll
      for (int w2 = 0; w2 < NW; ++w2) {
        const f32x4 o = reinterpret_cast<const f32x4*>(shm + (size_t)(w2 + NW * (UPW - 1)) * TILE)[lane];
        if (w2 == 0) {
          sacc = o;
        } else {
          sacc[0] += o[0];
          sacc[1] += o[1];
          sacc[2] += o[2];
          sacc[3] += o[3];
        }
      }
      // lane (j, g) holds L[row j][4g + v]
      lop[0] = u32x2{pack_bf16x2(sacc[0], sacc[1]), pack_bf16x2(sacc[2], sacc[3])};
      lopn[0] = neg_bf16x4(lop[0]);
    }
    lds_barrier();  // every wave's partial sums read: the slot KB may be refilled
    if (next) issue_tile(rb + 1, 2);
    uint8_t* crow = codes + (int64_t)row * ldc;
    uint16_t* qrow = qparams + (int64_t)row * ldq;
    auto unit = [&](int uu) {
      quant_unit<BITS, G, R>(x[uu], vop[uu], lopn, nullptr, ub + uu, N, g, crow, qrow);
      __builtin_amdgcn_sched_barrier(0);
    };
    unit(0);
    if (next) issue_tile(rb + 1, 3);
    unit(1);
    unit(2);
    if (next) {
      rotate_tile(0, C_T0{});
      issue_tile(rb + 1, 4);
    }
    unit(3);
    if (next) rotate_tile(1, C_T1{});
    unit(4);
    st8_pred(Lout + (int64_t)rb * 16 * ldl, (uint32_t)(16 * ldl * 2), (uint32_t)(((row - rb * 16) * ldl + 4 * g) * 2),
             lop[0], w == 0);
    __builtin_amdgcn_sched_barrier(0);
    if (next) {
      rotate_tile(2, C_T2{});
      rotate_tile(3, C_T3{});
    }
  };
#pragma unroll 1
  for (int b = 0; b < nblk - 1; ++b) block(std::true_type{}, b);
  block(std::false_type{}, nblk - 1);
}

// -------------------------------------------------------------------------------------
// Projection only (first pass of the two-pass encode).  Grid: ceil(rows / 16) workgroups
// of 4 waves; wave w sums 32-column chunks w, w + 4, ... of the row.  Uses V^T [R, N].
template <int R>
__global__ __launch_bounds__(256) void k_project(const uint16_t* __restrict__ X, int64_t ldx, int M,
                                                 int N, const uint16_t* __restrict__ Vt,
                                                 uint16_t* __restrict__ Lout, int64_t ldl) {
  constexpr int RT = R / 16, U = 4, NWV = 4;
  __shared__ f32x4 red[NWV * RT * 64];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int j = lane & 15, g = lane >> 4;
  const int row = blockIdx.x * 16 + j;
  const bool rv = row < M;
  const uint16_t* xrow = X + (int64_t)(rv ? row : 0) * ldx;
  const int NC = N / 32;
  f32x4 acc[RT];
#pragma unroll
  for (int t = 0; t < RT; ++t) acc[t] = zero4();
  for (int c = w; c < NC; c += NWV * U) {
    u32x4 xv[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int cc = c + NWV * u;
      xv[u] = (cc < NC && rv) ? ld16_stream(xrow + cc * 32 + 8 * g) : u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int cc = c + NWV * u;
      if (cc < NC) {
#pragma unroll
        for (int t = 0; t < RT; ++t) {
          const u32x4 a = ld16(Vt + (int64_t)(16 * t + j) * N + cc * 32 + 8 * g);
          acc[t] = mfma_16x16x32(a, xv[u], acc[t]);
        }
      }
    }
  }
#pragma unroll
  for (int t = 0; t < RT; ++t) red[(w * RT + t) * 64 + lane] = acc[t];
  __syncthreads();
  if (w == 0) {
#pragma unroll
    for (int t = 0; t < RT; ++t) {
      f32x4 s = red[t * 64 + lane];
#pragma unroll
      for (int w2 = 1; w2 < NWV; ++w2) {
        const f32x4 o = red[(w2 * RT + t) * 64 + lane];
        s[0] += o[0];
        s[1] += o[1];
        s[2] += o[2];
        s[3] += o[3];
      }
      if (rv)
        st8(Lout + (int64_t)row * ldl + 16 * t + 4 * g,
            u32x2{pack_bf16x2(s[0], s[1]), pack_bf16x2(s[2], s[3])});
    }
  }
}

// -------------------------------------------------------------------------------------
// Streaming residual + quantisation given L (second pass; the whole encode at rank 0).
// Grid: (ceil(rows / (64*RB)), units); a workgroup is 4 waves on the same unit, each wave
// walking RB row blocks, so the unit's V operands are loaded once per wave.  With OUTL,
// outlier columns are zeroed before the group statistics.
template <int BITS, int G, int R, int RB, bool OUTL>
__global__ __launch_bounds__(256) void k_quant(
    const uint16_t* __restrict__ X, int64_t ldx, int M, int N, const uint16_t* __restrict__ V,
    const uint16_t* __restrict__ Lin, int64_t ldl, uint8_t* __restrict__ codes, int64_t ldc,
    uint16_t* __restrict__ qparams, int64_t ldq, const int32_t* __restrict__ oidx, int nout) {
  constexpr int NP = 8 / BITS, CPG = G / 32, RT = R > 0 ? R / 16 : 1, E = G / 4;
  extern __shared__ uint32_t colmask[];
  if constexpr (OUTL) {
    for (int i = threadIdx.x; i < N / 32; i += blockDim.x) colmask[i] = 0u;
    __syncthreads();
    for (int k = threadIdx.x; k < nout; k += blockDim.x) {
      const int c = oidx[k];
      if (c >= 0 && c < N) atomicOr(&colmask[c >> 5], 1u << (c & 31));
    }
    __syncthreads();
  }
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int j = lane & 15, g = lane >> 4;
  const int u = blockIdx.y;
  u32x2 vop[NP][G / 16][RT];
  if constexpr (R > 0) {
#pragma unroll
    for (int p = 0; p < NP; ++p) load_vops<G, R>(V, unit_base(p, u, N, NP, G), j, g, vop[p]);
  }
  for (int b = 0; b < RB; ++b) {
    const int row = (blockIdx.x * RB + b) * 64 + w * 16 + j;
    if (row - j >= M) break;  // whole 16-row block past the end (uniform per wave)
    const int64_t rr = min(row, M - 1);
    u32x2 lopn[RT];  // -L
    if constexpr (R > 0) {
#pragma unroll
      for (int t = 0; t < RT; ++t) lopn[t] = neg_bf16x4(ld8(Lin + rr * ldl + 16 * t + 4 * g));
    }
    u32x4 x[NP][CPG];
#pragma unroll
    for (int p = 0; p < NP; ++p)
#pragma unroll
      for (int k = 0; k < CPG; ++k) x[p][k] = ld16_stream(X + rr * ldx + unit_base(p, u, N, NP, G) + E * g + 8 * k);
    quant_unit<BITS, G, R>(x, vop, lopn, OUTL ? colmask : nullptr, u, N, g, codes + rr * ldc,
                           qparams + rr * ldq);
  }
}

// -------------------------------------------------------------------------------------
// Two-pass encode over column slabs (rank 16/32 rows without a single-pass kernel).
//
// Pass 1, k_project_slab: grid (row groups, slabs); wave w of slab s owns the 256 columns
// c0 = 256*(8s + w) .. +255, whose V^T operands (8 K-steps of 32 columns x R/16 rank tiles)
// stay in registers.  Per 16-row block the wave's 16 x 512 B slice goes HBM -> registers ->
// a private LDS region (1 KB loads of two rows) and is read back in the MFMA layout; the eight
// waves' fp32 partials are summed in LDS in a fixed order, and the slab's partial L of the
// block is written to `part` (row r at part + r*ldp bytes, slab s at byte 4*R*s).  Columns
// past N contribute zero (their V^T operands are zero; their loads are clamped).
//
// Pass 1b, k_reduce_slabs: L = bf16(sum over slabs in order).
//
// Pass 2, k_quant_slab: residual and quantisation with L given.  Waves are independent (no
// barrier): global wave gw takes wave column gw % nwc (units 2*(gw % nwc) .. +1) and row
// range gw / nwc; its slice streams through a private LDS region as in k_encode_rows, with
// the next block's loads (and its L rows) in flight during the current block's quantisation.
template <int R, bool ROT, bool OUTL>
__global__ __launch_bounds__(512) void k_project_slab(const uint16_t* __restrict__ X, int64_t ldx, int M, int N,
                                                      const uint16_t* __restrict__ Vt,
                                                      unsigned char* __restrict__ part, int64_t ldp, int RBW,
                                                      const int32_t* __restrict__ oidx, int nout) {
  constexpr int RT = R / 16, NW = 8, CW = 256, PITCH = CW * 2 + 16, NLD = 8;
  __shared__ __attribute__((aligned(16))) unsigned char shm[NW * 16 * PITCH];
  __shared__ f32x4 red[2][NW][RT][64];
  extern __shared__ uint32_t pmask[];  // OUTL: N/32 words, outlier columns
  const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int j = lane & 15, g = lane >> 4;
  const int nrb = (M + 15) / 16;
  const int rb0 = blockIdx.x * RBW;
  if (rb0 >= nrb) return;  // whole workgroup
  const int nblk = min(RBW, nrb - rb0);
  const int s = blockIdx.y;
  const int c0 = CW * (NW * s + w);
  const bool live = c0 < N;  // wave-uniform
  unsigned char* region = shm + (size_t)w * 16 * PITCH;
  // ROT: the slice is rotated in place (WHT-128 per 128-column block) before use
  u32x4 wop[ROT ? 2 : 1][2];
  if constexpr (ROT) {
#pragma unroll
    for (int q0 = 0; q0 < 2; ++q0)
#pragma unroll
      for (int n = 0; n < 2; ++n) wop[q0][n] = wht_base_operand(j, g, q0, n != 0);
  }
  // V^T operands: vt[k][t] = Vt[16t + j][c0 + 32k + 8g .. +7] (zero past N)
  u32x4 vt[CW / 32][RT];
#pragma unroll
  for (int k = 0; k < CW / 32; ++k)
#pragma unroll
    for (int t = 0; t < RT; ++t) {
      const int c = c0 + 32 * k + 8 * g;
      vt[k][t] = c < N ? ld16(Vt + (int64_t)(16 * t + j) * N + c) : u32x4{0u, 0u, 0u, 0u};
    }
  // the lane's 8 columns of X as kept (ROT && OUTL: outlier columns zeroed before the rotation)
  uint32_t xkeep[4] = {~0u, ~0u, ~0u, ~0u};
  const int lr = lane >> 5;
  const uint32_t lcol = (uint32_t)min(c0 + (lane & 31) * 8, N - 8) * 2u;
  if constexpr (OUTL) {
    for (int i = threadIdx.x; i < N / 32; i += 512) pmask[i] = 0u;
    __syncthreads();
    for (int k = threadIdx.x; k < nout; k += 512) {
      const int c = oidx[k];
      if (c >= 0 && c < N) atomicOr(&pmask[c >> 5], 1u << (c & 31));
    }
    __syncthreads();
  }
  if constexpr (OUTL && ROT) {
    // the rotated format: the channels leave X before the rotation (the rotated columns are all
    // projected)
    const int c = (int)(lcol / 2u);  // 8 columns inside one mask word
    const uint32_t b8 = (pmask[c >> 5] >> (c & 31)) & 0xffu;
#pragma unroll
    for (int d = 0; d < 4; ++d)
      xkeep[d] = (((b8 >> (2 * d)) & 1u) ? 0u : 0x0000ffffu) | (((b8 >> (2 * d + 1)) & 1u) ? 0u : 0xffff0000u);
  } else if constexpr (OUTL) {
    // outlier columns meet zero V^T operands: the projection of Y with those columns zeroed
#pragma unroll
    for (int k = 0; k < CW / 32; ++k) {
      const int c = c0 + 32 * k + 8 * g;  // 8 columns inside one mask word
      const uint32_t b8 = c < N ? (pmask[c >> 5] >> (c & 31)) & 0xffu : 0u;
#pragma unroll
      for (int t = 0; t < RT; ++t)
#pragma unroll
        for (int d = 0; d < 4; ++d) {
          const uint32_t keep = (((b8 >> (2 * d)) & 1u) ? 0u : 0x0000ffffu) | (((b8 >> (2 * d + 1)) & 1u) ? 0u : 0xffff0000u);
          vt[k][t][d] &= keep;
        }
    }
  }
  // load i: rows 2i, 2i+1 of the block, lane l -> row 2i + l/32, bytes (l%32)*16 of the slice
  // (clamped to column N - 8 past the end: those columns meet zero operands)
  auto gaddr = [&](int rb, int i) {
    const int64_t row = min(rb * 16 + 2 * i + lr, M - 1);
    return reinterpret_cast<const unsigned char*>(X + row * ldx) + lcol;
  };
  u32x4 pf[NLD];
  auto issue = [&](int rb) {
#pragma unroll
    for (int i = 0; i < NLD; ++i) pf[i] = ld16_stream(gaddr(rb, i));
  };
  if (live) issue(rb0);
#pragma unroll 1
  for (int b = 0; b < nblk; ++b) {
    f32x4 acc[RT];
#pragma unroll
    for (int t = 0; t < RT; ++t) acc[t] = zero4();
    if (live) {
#pragma unroll
      for (int i = 0; i < NLD; ++i) {
        u32x4 v = pf[i];
        if constexpr (OUTL && ROT) v = u32x4{v[0] & xkeep[0], v[1] & xkeep[1], v[2] & xkeep[2], v[3] & xkeep[3]};
        *reinterpret_cast<u32x4*>(region + (2 * i + lr) * PITCH + (lane & 31) * 16) = v;
      }
      if constexpr (ROT) {
#pragma unroll
        for (int q = 0; q < CW / 128; ++q)
          if (c0 + 128 * q < N) wht128_lds(region + j * PITCH + (128 * q + 32 * g) * 2, wop);
      }
      u32x4 x[CW / 32];
#pragma unroll
      for (int k = 0; k < CW / 32; ++k) x[k] = *reinterpret_cast<const u32x4*>(region + j * PITCH + (32 * k + 8 * g) * 2);
      if (b + 1 < nblk) issue(rb0 + b + 1);
#pragma unroll
      for (int k = 0; k < CW / 32; ++k)
#pragma unroll
        for (int t = 0; t < RT; ++t) acc[t] = mfma_16x16x32(vt[k][t], x[k], acc[t]);
    }
#pragma unroll
    for (int t = 0; t < RT; ++t) red[b & 1][w][t][lane] = acc[t];
    lds_barrier();
    if (w < RT) {
      // wave t sums rank tile t over the eight waves; lane (j, g) holds L[row j][16t + 4g ..]
      const int t = w;
      f32x4 sum = red[b & 1][0][t][lane];
#pragma unroll
      for (int w2 = 1; w2 < NW; ++w2) {
        const f32x4 o = red[b & 1][w2][t][lane];
        sum[0] += o[0];
        sum[1] += o[1];
        sum[2] += o[2];
        sum[3] += o[3];
      }
      const int64_t row = min((rb0 + b) * 16 + j, M - 1);
      *reinterpret_cast<f32x4*>(part + row * ldp + 4 * R * s + (16 * t + 4 * g) * 4) = sum;
    }
  }
}

template <int R>
__global__ __launch_bounds__(256) void k_reduce_slabs(const unsigned char* __restrict__ part, int64_t ldp, int M,
                                                      int nslab, uint16_t* __restrict__ L, int64_t ldl) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;  // (row, 4 ranks)
  if (i >= (int64_t)M * (R / 4)) return;
  const int64_t row = i / (R / 4);
  const int q = (int)(i % (R / 4));
  const unsigned char* p = part + row * ldp + q * 16;
  f32x4 sum = *reinterpret_cast<const f32x4*>(p);
  for (int sl = 1; sl < nslab; ++sl) {
    const f32x4 o = *reinterpret_cast<const f32x4*>(p + 4 * R * sl);
    sum[0] += o[0];
    sum[1] += o[1];
    sum[2] += o[2];
    sum[3] += o[3];
  }
  *reinterpret_cast<u32x2*>(L + row * ldl + 4 * q) = u32x2{pack_bf16x2(sum[0], sum[1]), pack_bf16x2(sum[2], sum[3])};
}

template <int BITS, int G, int R, bool OUTL>
struct QuantSlab {
  static constexpr int NP = 8 / BITS, UPW = 2, NW = 8;
  static constexpr int PIECE = UPW * G * 2, PITCH = NP * PIECE + 16, PPL = 1024 / PIECE, LPL = 64 / PPL;
  static constexpr int RPL = PPL / NP, NLD = 16 / RPL;
  static constexpr size_t REGIONS = (size_t)NW * 16 * PITCH;
  static size_t bytes(int N) { return REGIONS + (OUTL ? (size_t)(N / 32) * 4 + (size_t)N * 2 : 0); }
  static_assert(PPL % NP == 0 && NLD * RPL == 16, "whole rows per load");
};

// Residual and quantisation pass of the column-slab encode (also the whole encode at rank 0).
// OUTL: outlier columns (oidx) are zeroed before the group statistics, and their bf16 values
// are written to the fp16 side columns from the slice in LDS (a wave-uniform loop over the
// wave's outlier columns; one range-checked 2-byte store per row).
template <int BITS, int G, int R, bool OUTL, bool ROT>
__global__ __launch_bounds__(512) void k_quant_slab(const uint16_t* __restrict__ X, int64_t ldx, int M, int N,
                                                    const uint16_t* __restrict__ V, const uint16_t* __restrict__ Lin,
                                                    int64_t ldl, uint8_t* __restrict__ codes, int64_t ldc,
                                                    uint16_t* __restrict__ qparams, int64_t ldq,
                                                    const int32_t* __restrict__ oidx, int nout,
                                                    uint16_t* __restrict__ side, int64_t ldside, int nranges,
                                                    int RBW) {
  using Qs = QuantSlab<BITS, G, R, OUTL>;
  constexpr int NP = Qs::NP, UPW = Qs::UPW, NW = Qs::NW, CPG = G / 32, RT = R > 0 ? R / 16 : 1, E = G / 4;
  constexpr int PIECE = Qs::PIECE, PITCH = Qs::PITCH, LPL = Qs::LPL, RPL = Qs::RPL, NLD = Qs::NLD;
  extern __shared__ __attribute__((aligned(16))) unsigned char shm[];
  uint32_t* colmask = reinterpret_cast<uint32_t*>(shm + Qs::REGIONS);  // OUTL: N/32 words
  int16_t* oslot = reinterpret_cast<int16_t*>(colmask + N / 32);      // OUTL: N entries
  if constexpr (OUTL) {
    for (int i = threadIdx.x; i < N / 32; i += blockDim.x) colmask[i] = 0u;
    for (int i = threadIdx.x; i < N; i += blockDim.x) oslot[i] = -1;
    __syncthreads();
    for (int k = threadIdx.x; k < nout; k += blockDim.x) {
      const int c = oidx[k];
      if (c >= 0 && c < N) {
        atomicOr(&colmask[c >> 5], 1u << (c & 31));
        oslot[c] = (int16_t)k;
      }
    }
    __syncthreads();  // the only barrier: waves are independent below
  }
  const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int j = lane & 15, g = lane >> 4;
  const int units = N / (G * NP), nwc = units / UPW;
  const int gw = blockIdx.x * NW + w;
  if (gw >= nranges * nwc) return;  // this wave only
  const int ub = UPW * (gw % nwc), rng = gw / nwc;
  const int nrb = (M + 15) / 16;
  const int rb0 = rng * RBW;
  if (rb0 >= nrb) return;
  const int nblk = min(RBW, nrb - rb0);
  unsigned char* region = shm + (size_t)w * 16 * PITCH;
  // ROT: the slice is rotated in place (WHT-128 per 128-column block of each plane) before use;
  // the host guarantees that the wave's columns of each plane start on a block boundary.  With
  // OUTL the side columns are taken from the slice and zeroed in it before the rotation.
  static_assert(!ROT || (UPW * G) % 128 == 0, "whole rotation blocks per wave and plane");
  u32x4 wop[ROT ? 2 : 1][2];
  if constexpr (ROT) {
#pragma unroll
    for (int q0 = 0; q0 < 2; ++q0)
#pragma unroll
      for (int n = 0; n < 2; ++n) wop[q0][n] = wht_base_operand(j, g, q0, n != 0);
  }

  u32x2 vop[UPW][NP][G / 16][RT];
  if constexpr (R > 0) {
#pragma unroll
    for (int uu = 0; uu < UPW; ++uu)
#pragma unroll
      for (int p = 0; p < NP; ++p) load_vops<G, R>(V, unit_base(p, ub + uu, N, NP, G), j, g, vop[uu][p]);
  }

  // load i: rows RPL*i .. of the block, lane l -> piece l/LPL (row RPL*i + (l/LPL)/NP, plane
  // (l/LPL)%NP) at byte (l%LPL)*16; rows past the end clamp to the last row
  const int lpc = lane / LPL, loff = (lane % LPL) * 16, lrow = lpc / NP;
  const uint32_t xlane = (uint32_t)unit_base(lpc % NP, ub, N, NP, G) * 2u + (uint32_t)loff;
  auto gaddr = [&](int rb, int i) {
    const int64_t row = min((int64_t)rb * 16 + RPL * i + lrow, (int64_t)M - 1);
    return reinterpret_cast<const unsigned char*>(X + row * ldx) + xlane;
  };
  u32x4 pf[NLD];
  u32x2 lnext[RT];
  auto issue = [&](int rb) {
#pragma unroll
    for (int i = 0; i < NLD; ++i) pf[i] = ld16_stream(gaddr(rb, i));
    if constexpr (R > 0) {
      const int64_t row = min(rb * 16 + j, M - 1);
#pragma unroll
      for (int t = 0; t < RT; ++t) lnext[t] = ld8(Lin + row * ldl + 16 * t + 4 * g);
    }
  };
  // side columns of the wave's units, read from the slice (lanes of quarter 0 store row j); a
  // wave-uniform loop over the wave's outlier columns, one range-checked 2-byte store per row.
  // zero: the columns are then zeroed in the slice (every lane of row j writes the same 0).
  auto side_pass = [&](int rb, int row, bool zero) {
    const __amdgpu_buffer_rsrc_t rs =
        uniform_rsrc(side + (int64_t)rb * 16 * ldside, (uint32_t)(16 * ldside * 2));
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      const int cb = unit_base(p, ub, N, NP, G);  // the wave's UPW*G contiguous columns of plane p
#pragma unroll 1
      for (int wd = 0; wd < UPW * G / 32; ++wd) {
        uint32_t bits = __builtin_amdgcn_readfirstlane(colmask[(cb >> 5) + wd]);
        while (bits != 0u) {
          const int e = __builtin_ctz(bits);
          bits &= bits - 1u;
          const int cl = 32 * wd + e;  // column within the wave's range
          const int k = oslot[cb + cl];
          uint16_t* px = reinterpret_cast<uint16_t*>(region + j * PITCH + p * PIECE + cl * 2);
          const uint32_t v = *px;
          const uint16_t h = (uint16_t)f16_bits(__uint_as_float(v << 16));
          __builtin_amdgcn_raw_buffer_store_b16(h, rs, g == 0 ? (uint32_t)(((row - rb * 16) * ldside + k) * 2) : 0x7ffffff0u,
                                                0, 0);
          if (zero) *px = 0;
        }
      }
    }
  };
  issue(rb0);
#pragma unroll 1
  for (int b = 0; b < nblk; ++b) {
    const int rb = rb0 + b;
    const int row = min(rb * 16 + j, M - 1);
#pragma unroll
    for (int i = 0; i < NLD; ++i)
      *reinterpret_cast<u32x4*>(region + (RPL * i + lrow) * PITCH + (lpc % NP) * PIECE + loff) = pf[i];
    if constexpr (OUTL && ROT) side_pass(rb, row, true);
    if constexpr (ROT) {
#pragma unroll
      for (int p = 0; p < NP; ++p)
#pragma unroll
        for (int q = 0; q < UPW * G / 128; ++q) wht128_lds(region + j * PITCH + p * PIECE + (128 * q + 32 * g) * 2, wop);
    }
    u32x4 x[UPW][NP][CPG];
#pragma unroll
    for (int uu = 0; uu < UPW; ++uu)
#pragma unroll
      for (int p = 0; p < NP; ++p)
#pragma unroll
        for (int k = 0; k < CPG; ++k)
          x[uu][p][k] = *reinterpret_cast<const u32x4*>(region + j * PITCH + p * PIECE + (uu * G + E * g + 8 * k) * 2);
    u32x2 lopn[RT];
    if constexpr (R > 0) {
#pragma unroll
      for (int t = 0; t < RT; ++t) lopn[t] = neg_bf16x4(lnext[t]);
    }
    if (b + 1 < nblk) issue(rb + 1);
    uint8_t* crow = codes + (int64_t)row * ldc;
    uint32_t qp[UPW];
#pragma unroll
    for (int uu = 0; uu < UPW; ++uu)
      qp[uu] = quant_unit_core<BITS, G, R>(x[uu], vop[uu], lopn, (OUTL && !ROT) ? colmask : nullptr, ub + uu, N, g,
                                           crow);
    if constexpr (NP == 2) {
      // the two units' (scale, zero) pairs of the row as one 16-byte store (see k_encode_rows)
      float a = __uint_as_float(qp[0]), bq = a, c = __uint_as_float(qp[1]), d = c;
      swap32(a, bq);
      swap32(c, d);
      st16_pred(qparams + (int64_t)rb * 16 * ldq, (uint32_t)(16 * ldq * 2),
                (uint32_t)(((row - rb * 16) * ldq + ub * NP * 2) * 2),
                u32x4{__float_as_uint(a), __float_as_uint(bq), __float_as_uint(c), __float_as_uint(d)}, g == 0);
    } else {
      // one plane: every lane of a row holds its unit's pair
      st8_pred(qparams + (int64_t)rb * 16 * ldq, (uint32_t)(16 * ldq * 2),
               (uint32_t)(((row - rb * 16) * ldq + ub * 2) * 2), u32x2{qp[0], qp[1]}, g == 0);
    }
    if constexpr (OUTL && !ROT) side_pass(rb, row, false);
  }
}

// Gather the outlier channels into fp16 side columns: side[r, k] = fp16(x[r, idx[k]]).
__global__ __launch_bounds__(256) void k_gather_side(const uint16_t* __restrict__ X, int64_t ldx, int M,
                                                     int N, const int32_t* __restrict__ oidx, int nout,
                                                     uint16_t* __restrict__ side, int64_t ldside) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (int64_t)M * nout) return;
  const int64_t r = i / nout;
  const int k = (int)(i - r * nout);
  const int c = oidx[k];
  const float v = (c >= 0 && c < N) ? __uint_as_float((uint32_t)X[r * ldx + c] << 16) : 0.f;
  side[r * ldside + k] = f16_bits(v);
}

// -------------------------------------------------------------------------------------
// host side

template <int BITS, int G, int R, int NW, int UPW, bool DB, int RBW>
static int launch_persist_rbw(const lrq_tensors* t, const void* x, int64_t ldx, hipStream_t s) {
  using Lds = PersistLds<BITS, G, R, NW, UPW>;
  // Wide waves keep their V operands in LDS so the double-buffered X tile fits in registers.
  constexpr bool VLDS = DB && (NW >= 16 || UPW * G * (8 / BITS) >= 512) && Lds::kVopBytes + Lds::kRedBytes <= 160 * 1024;
  const size_t shm = Lds::kRedBytes + (VLDS ? Lds::kVopBytes : 0);
  auto kern = k_encode_persist<BITS, G, R, NW, UPW, DB, VLDS, RBW>;
  if (shm > 64 * 1024) (void)hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)shm);
  const int nrb = (int)((t->rows + 15) / 16);
  LRQ_TRY(launch(kern, dim3((nrb + RBW - 1) / RBW), dim3(NW * 64), shm, s, (const uint16_t*)x, ldx,
                     (int)t->rows, (int)t->hidden, (const uint16_t*)t->V, (uint16_t*)t->L, t->ld_L,
                     (uint8_t*)t->codes, t->ld_codes, (uint16_t*)t->qparams, t->ld_qp));
  return LRQ_OK;
}

// Row blocks per workgroup: 4 when that still gives every CU a workgroup, else 1 (one
// workgroup of NW waves fits per CU).
template <int BITS, int G, int R, int NW, int UPW, bool DB>
static int launch_persist(const lrq_tensors* t, const void* x, int64_t ldx, hipStream_t s) {
  const int64_t nrb = (t->rows + 15) / 16;
  if (nrb >= 4 * (int64_t)cu_count()) return launch_persist_rbw<BITS, G, R, NW, UPW, DB, 4>(t, x, ldx, s);
  return launch_persist_rbw<BITS, G, R, NW, UPW, DB, 1>(t, x, ldx, s);
}

// k_encode_rows: one workgroup per CU, each walking ceil(row blocks / CUs) consecutive blocks.
template <int BITS, int G, int R, int UPW, bool OUTL>
static int launch_rows(const lrq_tensors* t, const void* x, int64_t ldx, hipStream_t s) {
  constexpr int NW = 8;
  using Re = RowsEnc<BITS, G, R, NW, UPW>;
  auto kern = k_encode_rows<BITS, G, R, NW, UPW, OUTL>;
  const size_t shm = Re::LDS + (OUTL ? (size_t)(t->hidden / 32) * 4 + (size_t)t->hidden * 2 : 0);
  const hipError_t e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)shm);
  if (e != hipSuccess) return (int)e;
  const int64_t nrb = (t->rows + 15) / 16, cus = cu_count();
  const int rbw = (int)((nrb + cus - 1) / cus);
  const int64_t wgs = (nrb + rbw - 1) / rbw;
  LRQ_TRY(launch(kern, dim3((unsigned)wgs), dim3(NW * 64), shm, s, (const uint16_t*)x, ldx, (int)t->rows,
                 (int)t->hidden, (const uint16_t*)t->V, (uint16_t*)t->L, t->ld_L, (uint8_t*)t->codes, t->ld_codes,
                 (uint16_t*)t->qparams, t->ld_qp, rbw, t->outlier_idx, (int)t->n_outlier, (uint16_t*)t->side,
                 t->ld_side));
  return LRQ_OK;
}

// k_encode_tiles (int4/g64, rank 16, NW*UPW units, no outlier channels): one workgroup per CU,
// each walking ceil(row blocks / CUs) consecutive blocks.  Returns 0 (nothing launched) when
// the shape does not fit or the device refuses the workgroup's 160 KB of LDS.
template <int BITS, int G, int R, bool ROT>
static int encode_tiles_dispatch(const lrq_tensors* t, const void* x, int64_t ldx, hipStream_t s, int* status) {
  if constexpr (BITS != 4 || G != 64 || R != 16) {
    return 0;
  } else {
    constexpr int UPW = 5;
    using Te = TilesEnc<UPW, ROT>;
    if (t->hidden != (int64_t)Te::NT * 128 || t->n_outlier > 0) return 0;
    if ((int64_t)16 * t->ld_L * 2 >= ((int64_t)1 << 31)) return 0;
    auto kern = k_encode_tiles<UPW, ROT>;
    if (hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)Te::LDS) != hipSuccess)
      return 0;
    const int64_t nrb = (t->rows + 15) / 16, cus = cu_count();
    const int rbw = (int)((nrb + cus - 1) / cus);
    const int64_t wgs = (nrb + rbw - 1) / rbw;
    *status = launch(kern, dim3((unsigned)wgs), dim3(Te::NW * 64), Te::LDS, s, (const uint16_t*)x, ldx, (int)t->rows,
                     (int)t->hidden, (const uint16_t*)t->V, (uint16_t*)t->L, t->ld_L, (uint8_t*)t->codes,
                     t->ld_codes, (uint16_t*)t->qparams, t->ld_qp, rbw);
    return 1;
  }
}

// The row-staged kernel with or without outlier channels (the side columns' 16-row stride must
// fit a buffer range and the mask and slot tables the LDS).
template <int BITS, int G, int R, int UPW>
static int launch_rows_any(const lrq_tensors* t, const void* x, int64_t ldx, hipStream_t s, int* status) {
  if (t->n_outlier == 0) {
    *status = launch_rows<BITS, G, R, UPW, false>(t, x, ldx, s);
    return 1;
  }
  using Re = RowsEnc<BITS, G, R, 8, UPW>;
  if (t->n_outlier > 32767 || (int64_t)16 * t->ld_side * 2 >= ((int64_t)1 << 31)) return 0;
  if (Re::LDS + (size_t)(t->hidden / 32) * 4 + (size_t)t->hidden * 2 > 160 * 1024) return 0;
  *status = launch_rows<BITS, G, R, UPW, true>(t, x, ldx, s);
  return 1;
}

// Returns 1 and launches when a single-pass kernel exists for this shape, else 0.
template <int BITS, int G, int R>
static int encode_persist_dispatch(const lrq_tensors* t, const void* x, int64_t ldx, hipStream_t s,
                                   int* status) {
  if constexpr (R != 16) {
    return 0;
  } else {
    constexpr int NP = 8 / BITS;
    // wide instantiations only where a wave's columns per unit (G*NP) keep it spill-free
    constexpr bool wide_ok = G * NP <= 128;
    const int64_t units = t->hidden / ((int64_t)G * NP);
    switch (units) {
      case 8:
        if (t->n_outlier > 0) return 0;
        *status = launch_persist<BITS, G, R, 4, 2, true>(t, x, ldx, s);
        return 1;
      case 16:
        // row-staged kernel (8 waves x 2 units; 16-byte qparams stores per row)
        if constexpr (BITS == 4 && G == 64) {
          if (t->ld_qp % 8 == 0 && aligned(t->qparams, 16)) return launch_rows_any<BITS, G, R, 2>(t, x, ldx, s, status);
        }
        if (t->n_outlier > 0) return 0;
        *status = launch_persist<BITS, G, R, 8, 2, true>(t, x, ldx, s);
        return 1;
      case 32:
        // row-staged kernel (8 waves x 4 units)
        if constexpr (BITS == 4 && G == 64) {
          if (t->ld_qp % 8 == 0 && aligned(t->qparams, 16)) return launch_rows_any<BITS, G, R, 4>(t, x, ldx, s, status);
        }
        if (t->n_outlier > 0) return 0;
        *status = launch_persist<BITS, G, R, 16, 2, true>(t, x, ldx, s);
        return 1;
      case 40:
        if (encode_tiles_dispatch<BITS, G, R, false>(t, x, ldx, s, status)) return 1;
        if constexpr (wide_ok) {
          if (t->n_outlier > 0) return 0;
          *status = launch_persist<BITS, G, R, 8, 5, false>(t, x, ldx, s);
          return 1;
        }
        return 0;
      default: return 0;
    }
  }
}

// Column-slab encode (see k_project_slab).  Rank > 0: projection partials, their reduction
// into L, then the quantisation pass; the slab partials of L live in the codes buffer until
// the quantisation pass overwrites it (row r's partials take the first nslab*4*R bytes of its
// codes row).  Rank 0: the quantisation pass alone (with outlier channels, it also writes the
// side columns).  Returns 0 when the shape does not fit this path.
template <int BITS, int G, int R, bool ROT>
static int encode_slabs(const lrq_tensors* t, const void* x, int64_t ldx, hipStream_t s, int* status) {
  constexpr int NP = 8 / BITS;
  const int M = (int)t->rows, N = (int)t->hidden;
  const int units = N / (G * NP);
  const int nslab = (N + 2047) / 2048;
  const bool outl = t->n_outlier > 0;
  if (units % 2 != 0 || N % 32 != 0) return 0;
  // rotated input: every wave's columns start on a 128-column block of their plane
  if (ROT && ((N / NP) % 128 != 0 || (2 * G) % 128 != 0 || (NP == 2 && G == 128))) return 0;
  if (outl && (t->n_outlier > 32767 || t->side == nullptr || t->outlier_idx == nullptr)) return 0;
  if (NP == 2 ? (t->ld_qp % 8 != 0 || !aligned(t->qparams, 16)) : (t->ld_qp % 4 != 0 || !aligned(t->qparams, 8))) return 0;
  if ((int64_t)16 * t->ld_qp * 2 >= ((int64_t)1 << 31)) return 0;
  if (outl && (int64_t)16 * t->ld_side * 2 >= ((int64_t)1 << 31)) return 0;
  const size_t shm = outl ? QuantSlab<BITS, G, R, true>::bytes(N) : QuantSlab<BITS, G, R, false>::bytes(N);
  if (shm > 160 * 1024) return 0;
  const int cus = cu_count();
  const int nrb = (M + 15) / 16;
  if constexpr (R > 0) {
    const int64_t ldp = t->ld_codes;  // bytes
    if ((int64_t)nslab * 4 * R > (int64_t)N * BITS / 8 || ldp % 16 != 0 || !aligned(t->codes, 16)) return 0;
    if (t->ld_L % 4 != 0 || !aligned(t->L, 8)) return 0;
    // pass 1: about one workgroup per CU over (row groups, slabs)
    const int per1 = std::max(1, cus / nslab);
    const int rbw1 = (nrb + per1 - 1) / per1;
    int st = outl ? launch((k_project_slab<R, ROT, true>), dim3((nrb + rbw1 - 1) / rbw1, nslab), dim3(512),
                           (size_t)(N / 32) * 4, s, (const uint16_t*)x, ldx, M, N, (const uint16_t*)t->Vt,
                           (unsigned char*)t->codes, ldp, rbw1, t->outlier_idx, (int)t->n_outlier)
                  : launch((k_project_slab<R, ROT, false>), dim3((nrb + rbw1 - 1) / rbw1, nslab), dim3(512), 0, s,
                           (const uint16_t*)x, ldx, M, N, (const uint16_t*)t->Vt, (unsigned char*)t->codes, ldp,
                           rbw1, nullptr, 0);
    if (st) { *status = st; return 1; }
    const int64_t nred = (int64_t)M * (R / 4);
    st = launch((k_reduce_slabs<R>), dim3((unsigned)((nred + 255) / 256)), dim3(256), 0, s,
                (const unsigned char*)t->codes, ldp, M, nslab, (uint16_t*)t->L, t->ld_L);
    if (st) { *status = st; return 1; }
  }
  // quantisation pass: 8 independent waves per workgroup, one workgroup per CU
  const int nwc = units / 2;
  const int nranges = std::max(1, std::min(nrb, cus * 8 / nwc));
  const int rbw2 = (nrb + nranges - 1) / nranges;
  const int waves = nranges * nwc;
  auto quant = [&](auto kern) {
    if (shm > 64 * 1024) (void)hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)shm);
    *status = launch(kern, dim3((waves + 7) / 8), dim3(512), shm, s, (const uint16_t*)x, ldx, M, N,
                     (const uint16_t*)t->V, (const uint16_t*)t->L, t->ld_L, (uint8_t*)t->codes, t->ld_codes,
                     (uint16_t*)t->qparams, t->ld_qp, t->outlier_idx, (int)t->n_outlier, (uint16_t*)t->side,
                     t->ld_side, nranges, rbw2);
  };
  if constexpr (ROT) {
    if constexpr (NP == 2 && G == 128) return 0;  // not built (its registers would spill)
    else if (outl) quant(k_quant_slab<BITS, G, R, true, true>);
    else quant(k_quant_slab<BITS, G, R, false, true>);
  } else {
    if (outl) {
      quant(k_quant_slab<BITS, G, R, true, false>);
    } else {
      quant(k_quant_slab<BITS, G, R, false, false>);
    }
  }
  return 1;
}

template <int BITS, int G, int R>
static int encode_twopass(const lrq_tensors* t, const void* x, int64_t ldx, hipStream_t s) {
  const int M = (int)t->rows, N = (int)t->hidden;
  constexpr int NP = 8 / BITS, RB = 4;
  {
    int st = 0;
    if (encode_slabs<BITS, G, R, false>(t, x, ldx, s, &st)) return st;
  }
  // the fallback projection reads V^T straight from memory: no outlier mask there
  if (R > 0 && t->n_outlier > 0) return LRQ_ERR_UNSUPPORTED;
  if constexpr (R > 0) {
    LRQ_TRY(launch((k_project<R>), dim3((M + 15) / 16), dim3(256), 0, s, (const uint16_t*)x, ldx, M, N,
                       (const uint16_t*)t->Vt, (uint16_t*)t->L, t->ld_L));
  }
  const int units = N / (G * NP);
  dim3 grid((M + 64 * RB - 1) / (64 * RB), units);
  if (t->n_outlier > 0) {
    LRQ_TRY(launch((k_quant<BITS, G, R, RB, true>), grid, dim3(256), (size_t)(N / 32) * 4, s,
                       (const uint16_t*)x, ldx, M, N, (const uint16_t*)t->V, (const uint16_t*)t->L, t->ld_L,
                       (uint8_t*)t->codes, t->ld_codes, (uint16_t*)t->qparams, t->ld_qp, t->outlier_idx,
                       t->n_outlier));
    const int64_t n = (int64_t)M * t->n_outlier;
    LRQ_TRY(launch(k_gather_side, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, (const uint16_t*)x,
                       ldx, M, N, t->outlier_idx, t->n_outlier, (uint16_t*)t->side, t->ld_side));
  } else {
    LRQ_TRY(launch((k_quant<BITS, G, R, RB, false>), grid, dim3(256), 0, s, (const uint16_t*)x, ldx, M, N,
                       (const uint16_t*)t->V, (const uint16_t*)t->L, t->ld_L, (uint8_t*)t->codes, t->ld_codes,
                       (uint16_t*)t->qparams, t->ld_qp, nullptr, 0));
  }
  return LRQ_OK;
}

template <int BITS, int G, int R>
static int encode_impl(const lrq_tensors* t, const void* x, int64_t ldx, hipStream_t s, int force_twopass) {
  int st = 0;
  if (t->flags & LRQ_FLAG_HADAMARD) {
    // rotated format: the single-pass tile kernel, or the column-slab passes, rotate X in LDS
    // as they read it
    if (!force_twopass && encode_tiles_dispatch<BITS, G, R, true>(t, x, ldx, s, &st)) return st;
    if (R > 0 && t->Vt == nullptr) return LRQ_ERR_NULL;
    if (encode_slabs<BITS, G, R, true>(t, x, ldx, s, &st)) return st;
    return LRQ_ERR_UNSUPPORTED;
  }
  if (!force_twopass && encode_persist_dispatch<BITS, G, R>(t, x, ldx, s, &st)) return st;
  if (R > 0 && t->Vt == nullptr) return LRQ_ERR_NULL;  // the two-pass projection reads V^T
  return encode_twopass<BITS, G, R>(t, x, ldx, s);
}

static int encode_entry(const lrq_tensors* t, const void* x, int64_t ldx, void* stream, int force_twopass) {
  int st = validate_tensors(t);
  if (st) return st;
  if (x == nullptr) return LRQ_ERR_NULL;
  if (ldx < t->hidden) return LRQ_ERR_SHAPE;
  if ((ldx % 8) != 0 || !aligned(x, 16)) return LRQ_ERR_ALIGN;
  if (t->rows == 0) return LRQ_OK;
  hipStream_t s = (hipStream_t)stream;
  switch (format_key(t->bits, t->group, t->rank)) {
    case format_key(4, 64, 0): return encode_impl<4, 64, 0>(t, x, ldx, s, force_twopass);
    case format_key(4, 64, 16): return encode_impl<4, 64, 16>(t, x, ldx, s, force_twopass);
    case format_key(4, 64, 32): return encode_impl<4, 64, 32>(t, x, ldx, s, force_twopass);
    case format_key(4, 128, 0): return encode_impl<4, 128, 0>(t, x, ldx, s, force_twopass);
    case format_key(4, 128, 16): return encode_impl<4, 128, 16>(t, x, ldx, s, force_twopass);
    case format_key(8, 64, 0): return encode_impl<8, 64, 0>(t, x, ldx, s, force_twopass);
    case format_key(8, 64, 16): return encode_impl<8, 64, 16>(t, x, ldx, s, force_twopass);
    case format_key(8, 128, 0): return encode_impl<8, 128, 0>(t, x, ldx, s, force_twopass);
    case format_key(8, 128, 16): return encode_impl<8, 128, 16>(t, x, ldx, s, force_twopass);
    default: return LRQ_ERR_UNSUPPORTED;
  }
}

}  // namespace lrq

extern "C" int lrq_encode(const lrq_tensors* t, const void* x, int64_t ldx, void* stream) {
  return lrq::encode_entry(t, x, ldx, stream, 0);
}

extern "C" int lrq_encode_twopass(const lrq_tensors* t, const void* x, int64_t ldx, void* stream) {
  return lrq::encode_entry(t, x, ldx, stream, 1);
}
