// Group-mode decode and the fused elementwise consumers (SiLU backward, GELU backward,
// elementwise product).  One streaming pass: codes, qparams and L are read once, the
// low-rank term L V^T is rebuilt on MFMA in the lanes that own the columns, and the
// epilogue either stores x_hat (bf16) or applies the consumer with the
// upstream gradient, so the full-precision activation never goes back to HBM.
//
// Work split: a workgroup is NW waves on NW consecutive units (G columns of every packing
// plane, see lrq_common.h) of the same rows; each wave keeps its unit's V operands in
// registers and walks its row blocks, prefetching the next block's codes, qparams and L
// while it computes the current.
#include "lrq_common.h"
#include "lrq_host.h"
#include "lrq_dequant.h"
#include "lrq_whtop.h"
#include "lrq_math.h"

#include <algorithm>
#include <type_traits>

namespace lrq {

// ------------------------------------------------------------------ epilogues
// An epilogue maps 8 consecutive reconstructed values of a row (fp32, before the bf16
// rounding that defines x_hat) to the 8 bf16 it stores.  Consumers that read a second
// tensor (kIn) get its 8 matching bf16 as a vector that the kernel prefetched together with
// the codes: on gfx9 one in-order counter tracks loads and stores, so a load issued after
// a row block's stores could only be consumed once those stores had completed.
struct EpiStore {
  static constexpr bool kIn = false, kRot = false;
  uint16_t* out;
  int64_t ld;
  __device__ __forceinline__ const uint16_t* in_row(int64_t) const { return nullptr; }
  __device__ __forceinline__ uint16_t* out_row(int64_t r) const { return out + r * ld; }
  __host__ __device__ __forceinline__ int64_t in_ld() const { return 0; }
  __host__ __device__ __forceinline__ int64_t out_ld() const { return ld; }
  __device__ __forceinline__ u32x4 apply(const float* xh, u32x4) const { return pack8(xh); }
};

// EpiStore followed by the inverse of the rotated format's rotation: the row kernel rotates
// each 128-column block of the bf16 output tile in LDS before storing it (x = WHT(bf16(Y'))).
struct EpiStoreRot : EpiStore {
  static constexpr bool kRot = true;
};

// A consumer on the rotated format: the compute pass stores bf16(Y') like EpiStore, the
// rotation pass applies the consumer to the rotated values (x_hat = bf16(WHT(bf16(Y'))), the
// decode's result) with the matching second-tensor values, and stores that.
template <class Inner>
struct EpiRot : Inner {
  static constexpr bool kRot = true;
  __device__ __forceinline__ u32x4 apply(const float* xh, u32x4) const { return pack8(xh); }
  __device__ __forceinline__ u32x4 rot_apply(const float* y, u32x4 in) const { return Inner::apply(y, in); }
};

// silu_backward.py:6-8 on x = bf16(x_hat), fp32 (lrq_math.h).
struct EpiSilu {
  static constexpr bool kIn = true, kRot = false;
  const uint16_t* dy;
  int64_t lddy;
  uint16_t* dx;
  int64_t lddx;
  __device__ __forceinline__ const uint16_t* in_row(int64_t r) const { return dy + r * lddy; }
  __device__ __forceinline__ uint16_t* out_row(int64_t r) const { return dx + r * lddx; }
  __host__ __device__ __forceinline__ int64_t in_ld() const { return lddy; }
  __host__ __device__ __forceinline__ int64_t out_ld() const { return lddx; }
  __device__ __forceinline__ u32x4 apply(const float* xh, u32x4 dyv) const {
    float d[8], o[8], x[8];
    unpack8(dyv, d);
#pragma unroll
    for (int e = 0; e < 8; e += 2) {  // x = bf16(x_hat), two per conversion
      x[e] = xh[e];
      x[e + 1] = xh[e + 1];
      bf16_roundtrip2(x[e], x[e + 1]);
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = silu_bwd_f32(x[e], d[e]);
    return pack8(o);
  }
};

// gelu_backward.py:14-21 (tanh approximation) on x = bf16(x_hat), fp32 (lrq_math.h).
struct EpiGelu {
  static constexpr bool kIn = true, kRot = false;
  const uint16_t* dy;
  int64_t lddy;
  uint16_t* dx;
  int64_t lddx;
  __device__ __forceinline__ const uint16_t* in_row(int64_t r) const { return dy + r * lddy; }
  __device__ __forceinline__ uint16_t* out_row(int64_t r) const { return dx + r * lddx; }
  __host__ __device__ __forceinline__ int64_t in_ld() const { return lddy; }
  __host__ __device__ __forceinline__ int64_t out_ld() const { return lddx; }
  __device__ __forceinline__ u32x4 apply(const float* xh, u32x4 dyv) const {
    float d[8], o[8], x[8];
    unpack8(dyv, d);
#pragma unroll
    for (int e = 0; e < 8; e += 2) {  // x = bf16(x_hat), two per conversion
      x[e] = xh[e];
      x[e + 1] = xh[e + 1];
      bf16_roundtrip2(x[e], x[e + 1]);
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = gelu_bwd_f32(x[e], d[e]);
    return pack8(o);
  }
};

// extraction_fuse_hadamard.py:5-6: x * y.
struct EpiMul {
  static constexpr bool kIn = true, kRot = false;
  const uint16_t* y;
  int64_t ldy;
  uint16_t* out;
  int64_t ldo;
  __device__ __forceinline__ const uint16_t* in_row(int64_t r) const { return y + r * ldy; }
  __device__ __forceinline__ uint16_t* out_row(int64_t r) const { return out + r * ldo; }
  __host__ __device__ __forceinline__ int64_t in_ld() const { return ldy; }
  __host__ __device__ __forceinline__ int64_t out_ld() const { return ldo; }
  __device__ __forceinline__ u32x4 apply(const float* xh, u32x4 yv) const {
    float a[8], o[8], x[8];
    unpack8(yv, a);
#pragma unroll
    for (int e = 0; e < 8; e += 2) {  // x = bf16(x_hat), two per conversion
      x[e] = xh[e];
      x[e + 1] = xh[e + 1];
      bf16_roundtrip2(x[e], x[e + 1]);
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = x[e] * a[e];
    return pack8(o);
  }
};

// ------------------------------------------------------------------ kernel
// Per-row-block inputs of one lane: its G/4 code bytes, the unit's NP (scale, zero) pairs,
// the L operand of its row and, for consumers that read a second tensor, its G/4 columns of
// that tensor in every plane.
template <int BITS, int G, int R, bool IN>
struct DecIn {
  u32x4 cb[G / 64];
  uint32_t qp[8 / BITS];
  u32x2 lop[R > 0 ? R / 16 : 1];
  u32x4 ein[IN ? 8 / BITS : 1][IN ? G / 32 : 1];
};

// Grid: (ceil(row blocks / RBW), ceil(units / NW)); NW waves; wave w owns unit
// blockIdx.y * NW + w and walks row blocks blockIdx.x * RBW + b, b < RBW, keeping the
// inputs of the next PD blocks in flight while it reconstructs and stores block b.  The waves of a
// workgroup work on consecutive units of the same rows, so at any time a workgroup writes
// NW * G * 2 contiguous bytes per row and plane (DRAM-page friendly), while each wave
// reuses its unit's V operands for all its row blocks.
template <int BITS, int G, int R, bool OUTL, int NW, int RBW, int PD, class EPI>
__global__ __launch_bounds__(NW * 64) void k_decode(
    const uint8_t* __restrict__ codes, int64_t ldc, const uint16_t* __restrict__ qparams, int64_t ldq,
    const uint16_t* __restrict__ Lin, int64_t ldl, const uint16_t* __restrict__ V, int M, int N,
    const int32_t* __restrict__ oidx, int nout, const uint16_t* __restrict__ side, int64_t ldside,
    EPI epi) {
  constexpr int NP = 8 / BITS, RT = R > 0 ? R / 16 : 1, E = G / 4;
  extern __shared__ uint32_t smem[];
  uint32_t* colmask = smem;                                    // N/32 words
  int16_t* slot = reinterpret_cast<int16_t*>(smem + N / 32);  // N entries
  if constexpr (OUTL) {
    for (int i = threadIdx.x; i < N / 32; i += blockDim.x) colmask[i] = 0u;
    for (int i = threadIdx.x; i < N; i += blockDim.x) slot[i] = -1;
    __syncthreads();
    for (int k = threadIdx.x; k < nout; k += blockDim.x) {
      const int c = oidx[k];
      if (c >= 0 && c < N) {
        atomicOr(&colmask[c >> 5], 1u << (c & 31));
        slot[c] = (int16_t)k;
      }
    }
    __syncthreads();
  }
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int j = lane & 15, g = lane >> 4;
  const int u = blockIdx.y * NW + w;
  if (u >= N / (G * NP)) return;  // tail workgroup of a row: idle wave (no barrier follows)
  const int nrb = (M + 15) / 16;

  u32x2 vop[NP][G / 16][RT];
  if constexpr (R > 0) {
#pragma unroll
    for (int p = 0; p < NP; ++p) load_vops<G, R>(V, unit_base(p, u, N, NP, G), j, g, vop[p]);
  }

  using In = DecIn<BITS, G, R, EPI::kIn>;
  auto load = [&](In& in, int rb) __attribute__((always_inline)) {
    const int64_t row = min(rb * 16 + j, M - 1);
    const uint8_t* cp = codes + row * ldc + u * G + E * g;
#pragma unroll
    for (int i = 0; i < G / 64; ++i) in.cb[i] = ld16_stream(cp + 16 * i);
    const uint16_t* qpp = qparams + row * ldq + u * NP * 2;
    if constexpr (NP == 2) {
      const u32x2 v = ld8(qpp);
      in.qp[0] = v[0];
      in.qp[1] = v[1];
    } else {
      in.qp[0] = ld4(qpp);
    }
    if constexpr (R > 0) {
#pragma unroll
      for (int t = 0; t < RT; ++t) in.lop[t] = ld8(Lin + row * ldl + 16 * t + 4 * g);
    }
    if constexpr (EPI::kIn) {
      const uint16_t* ir = epi.in_row(row);
#pragma unroll
      for (int p = 0; p < NP; ++p)
#pragma unroll
        for (int k = 0; k < G / 32; ++k) in.ein[p][k] = ld16_stream(ir + unit_base(p, u, N, NP, G) + E * g + 8 * k);
    }
  };

  auto compute = [&](const In& in, int rb) __attribute__((always_inline)) {
    const int64_t rr = min(rb * 16 + j, M - 1);
    uint16_t* orow = epi.out_row(rr);
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      float xh[E];
      reconstruct_plane<BITS, G, R>(in.cb, in.qp[p], p, vop[p], in.lop, xh);
      const int c0 = unit_base(p, u, N, NP, G) + E * g;
      if constexpr (OUTL) {
        const uint32_t mbits = colmask[c0 >> 5] >> (c0 & 31);
        if (mbits != 0u) {
#pragma unroll
          for (int e = 0; e < E; ++e)
            if ((mbits >> e) & 1u) xh[e] = f16_val(side[rr * ldside + slot[c0 + e]]);
        }
      }
#pragma unroll
      for (int k = 0; k < E / 8; ++k) st16(orow + c0 + 8 * k, epi.apply(xh + 8 * k, in.ein[EPI::kIn ? p : 0][EPI::kIn ? k : 0]));
    }
  };

  const int rb0 = blockIdx.x * RBW;
  if (rb0 >= nrb) return;
  // The inputs of the first PD blocks are requested up front; block b + PD is requested
  // before block b is reconstructed and stored (PD + 1 register buffers, indices fixed after
  // unrolling).  On gfx9 one in-order counter tracks loads and stores, so waiting for a load
  // issued after a store also waits for that store: PD >= RBW (every load issued before the
  // first store) is the fastest form measured on MI355X.  With RBW and PD compile-time
  // constants and no branch in the body every wait count is exact.  Blocks past the end
  // (tail workgroup only) repeat the last row block, rewriting the same bytes.
  In in[PD < RBW ? PD + 1 : RBW];
  constexpr int NB = PD < RBW ? PD + 1 : RBW;
#pragma unroll
  for (int b = 0; b < PD && b < RBW; ++b) load(in[b % NB], min(rb0 + b, nrb - 1));
#pragma unroll
  for (int b = 0; b < RBW; ++b) {
    if (b + PD < RBW) load(in[(b + PD) % NB], min(rb0 + b + PD, nrb - 1));
    __builtin_amdgcn_sched_barrier(0);
    compute(in[b % NB], min(rb0 + b, nrb - 1));
    __builtin_amdgcn_sched_barrier(0);
  }
}

// ------------------------------------------------------------------ staged kernel
// Same work split and arithmetic as k_decode, but each row block's codes, qparams and L are
// loaded cooperatively: the workgroup's lanes read the tile with contiguous 16-byte (codes)
// and 8-byte (qparams, L) loads, whole row segments at a time, pass it through LDS (two
// slots, one barrier per block), and every wave then reads its unit back in the
// reconstruction layout.  Per-lane loads of the unit layout gather 16 rows x 64 bytes per
// instruction; on MI355X those fragmented reads neither stream at full rate nor overlap
// the stores (a decode with its reads removed runs 30 % faster, one with its stores removed
// reads at under half the bandwidth of contiguous reads).
// Every load of the workgroup's RBW blocks is issued before the first store, as in
// k_decode.  Waves past the last unit of a row take part in the loads and barriers only.
template <int BITS, int G, int R, int NW>
struct StagedTile {
  static constexpr int NP = 8 / BITS, T = NW * 64;
  static constexpr int CROW = NW * G;                     // code bytes per tile row
  static constexpr int CCH = CROW;                        // 16-byte code chunks per tile (16 rows)
  static constexpr int CPT = CCH / T;                     // per thread
  static constexpr int QROW = NW * NP * 4;                // qparam bytes per tile row
  static constexpr int QCH = 2 * QROW;                    // 8-byte qparam chunks per tile
  static constexpr int LROW = R * 2;                      // L bytes per row
  static constexpr int LCH = 2 * LROW;                    // 8-byte L chunks per tile
  static constexpr int QOFF = 16 * CROW, LOFF = QOFF + 16 * QROW;
  static constexpr int SLOT = LOFF + 16 * LROW;           // bytes per slot
  static_assert(CCH % T == 0 && CPT >= 1, "code tile split");
  static_assert(QCH + LCH <= T, "qparam / L tile split");
  static_assert(SLOT % 16 == 0 && QROW % 8 == 0, "alignment");
};

template <int BITS, int G, int R, int NW, int RBW, class EPI>
__global__ __launch_bounds__(NW * 64) void k_decode_staged(
    const uint8_t* __restrict__ codes, int64_t ldc, const uint16_t* __restrict__ qparams, int64_t ldq,
    const uint16_t* __restrict__ Lin, int64_t ldl, const uint16_t* __restrict__ V, int M, int N, EPI epi) {
  using Tl = StagedTile<BITS, G, R, NW>;
  constexpr int NP = 8 / BITS, RT = R > 0 ? R / 16 : 1, E = G / 4, T = Tl::T;
  extern __shared__ __attribute__((aligned(16))) unsigned char sm[];  // [2][SLOT]
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int j = lane & 15, g = lane >> 4;
  const int units = N / (G * NP);
  const int u0 = blockIdx.y * NW, u = u0 + w;
  const int nu = min(NW, units - u0);  // units present in this workgroup
  const bool active = u < units;
  const int nrb = (M + 15) / 16;
  const int rb0 = blockIdx.x * RBW;
  if (rb0 >= nrb) return;  // whole workgroup (no barrier reached)

  u32x2 vop[NP][G / 16][RT];
  if constexpr (R > 0) {
    if (active) {
#pragma unroll
      for (int p = 0; p < NP; ++p) load_vops<G, R>(V, unit_base(p, u, N, NP, G), j, g, vop[p]);
    }
  }

  struct In {
    u32x4 c[Tl::CPT];
    u32x2 ql;  // this thread's qparam or L chunk (if any)
    u32x4 ein[EPI::kIn ? NP : 1][EPI::kIn ? G / 32 : 1];
  };
  // chunk geometry of this thread (fixed over blocks)
  const int qk = tid, lk = tid - Tl::QCH;
  const bool has_q = qk < Tl::QCH && (qk % (Tl::QROW / 8)) * 8 < nu * NP * 4;
  const bool has_l = R > 0 && lk >= 0 && lk < Tl::LCH;
  auto load = [&](In& in, int rb) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < Tl::CPT; ++i) {
      const int k = tid + T * i, r = k / (Tl::CROW / 16), c16 = k % (Tl::CROW / 16);
      const int64_t row = min(rb * 16 + r, M - 1);
      if (c16 * 16 < nu * G) in.c[i] = ld16_stream(codes + row * ldc + (int64_t)u0 * G + c16 * 16);
    }
    if (has_q) {
      const int r = qk / (Tl::QROW / 8), c8 = qk % (Tl::QROW / 8);
      const int64_t row = min(rb * 16 + r, M - 1);
      in.ql = ld8(reinterpret_cast<const uint8_t*>(qparams) + (row * ldq + (int64_t)u0 * NP * 2) * 2 + c8 * 8);
    } else if (has_l) {
      const int r = lk / (Tl::LROW / 8), c8 = lk % (Tl::LROW / 8);
      const int64_t row = min(rb * 16 + r, M - 1);
      in.ql = ld8(reinterpret_cast<const uint8_t*>(Lin) + row * ldl * 2 + c8 * 8);
    }
    if constexpr (EPI::kIn) {
      if (active) {
        const uint16_t* ir = epi.in_row(min(rb * 16 + j, M - 1));
#pragma unroll
        for (int p = 0; p < NP; ++p)
#pragma unroll
          for (int k = 0; k < G / 32; ++k) in.ein[p][k] = ld16_stream(ir + unit_base(p, u, N, NP, G) + E * g + 8 * k);
      }
    }
  };

  In in[RBW];
#pragma unroll
  for (int b = 0; b < RBW; ++b) load(in[b], min(rb0 + b, nrb - 1));
  __builtin_amdgcn_sched_barrier(0);

#pragma unroll
  for (int b = 0; b < RBW; ++b) {
    const int rb = min(rb0 + b, nrb - 1);
    unsigned char* slot = sm + (b & 1) * Tl::SLOT;
#pragma unroll
    for (int i = 0; i < Tl::CPT; ++i) {
      const int k = tid + T * i, r = k / (Tl::CROW / 16), c16 = k % (Tl::CROW / 16);
      if (c16 * 16 < nu * G) *reinterpret_cast<u32x4*>(slot + r * Tl::CROW + c16 * 16) = in[b].c[i];
    }
    if (has_q) {
      const int r = qk / (Tl::QROW / 8), c8 = qk % (Tl::QROW / 8);
      *reinterpret_cast<u32x2*>(slot + Tl::QOFF + r * Tl::QROW + c8 * 8) = in[b].ql;
    } else if (has_l) {
      const int r = lk / (Tl::LROW / 8), c8 = lk % (Tl::LROW / 8);
      *reinterpret_cast<u32x2*>(slot + Tl::LOFF + r * Tl::LROW + c8 * 8) = in[b].ql;
    }
    lds_barrier();
    if (active) {
      u32x4 cb[G / 64];
#pragma unroll
      for (int i = 0; i < G / 64; ++i)
        cb[i] = *reinterpret_cast<const u32x4*>(slot + j * Tl::CROW + w * G + E * g + 16 * i);
      uint32_t qp[NP];
      if constexpr (NP == 2) {
        const u32x2 q = *reinterpret_cast<const u32x2*>(slot + Tl::QOFF + j * Tl::QROW + w * 8);
        qp[0] = q[0];
        qp[1] = q[1];
      } else {
        qp[0] = *reinterpret_cast<const uint32_t*>(slot + Tl::QOFF + j * Tl::QROW + w * 4);
      }
      u32x2 lop[RT];
      if constexpr (R > 0) {
#pragma unroll
        for (int t = 0; t < RT; ++t)
          lop[t] = *reinterpret_cast<const u32x2*>(slot + Tl::LOFF + j * Tl::LROW + 32 * t + 8 * g);
      }
      const int64_t rr = min(rb * 16 + j, M - 1);
      uint16_t* orow = epi.out_row(rr);
#pragma unroll
      for (int p = 0; p < NP; ++p) {
        float xh[E];
        reconstruct_plane<BITS, G, R>(cb, qp[p], p, vop[p], lop, xh);
        const int c0 = unit_base(p, u, N, NP, G) + E * g;
#pragma unroll
        for (int k = 0; k < E / 8; ++k)
          st16(orow + c0 + 8 * k, epi.apply(xh + 8 * k, in[b].ein[EPI::kIn ? p : 0][EPI::kIn ? k : 0]));
      }
    }
  }
}

// ------------------------------------------------------------------ row-persistent kernel
// Decode and the fused elementwise consumers at about one workgroup per CU.  Same per-block
// arithmetic and input staging as k_decode_staged; the difference is the full-precision side.
// Each wave writes its reconstructed (or consumed) unit, 16 rows x NP planes x G columns in
// the MFMA layout, into an LDS output tile, and after the next barrier the workgroup stores the
// tile as whole row segments: one 16-byte vector per lane, nu*G*2 contiguous bytes per row and
// plane (nu = units of the workgroup).  A consumer's second tensor (dY) comes the opposite way:
// whole row segments into an LDS input tile, read back in the MFMA layout.  The MFMA layout
// moves 4 x 16 B pieces of 16 rows per instruction; on MI355X such partial-line traffic, and a
// second workgroup interleaving its own on the CU, cost about a third of the decode's time.
//
// Pipeline (one barrier per row block b): write block b's staged inputs into slot b&1 ->
// barrier -> store the output tile of block b-1 (slot (b-1)&1) -> compute block b into output
// slot b&1.  A slot is rewritten two blocks later, after a barrier that every wave reaches only
// once its reads of that slot have returned.  All input loads of the workgroup's RBW blocks are
// issued before the first store (loads and stores share one in-order counter on gfx9).  Waves
// past the last unit of the row take part in the loads, barriers and stores only.
//
// OUTL (rank 0, at most kSideMax outlier channels): the fp16 side columns of each block are
// staged with the codes, and reconstructed values of outlier columns are replaced by them.
static constexpr int kSideMax = 64;
// Row blocks the plain decode moves from each odd-XCD workgroup to its even-XCD partner (see
// k_decode_rows): 2 of 16, for the odd XCDs' ~11 % lower decode rate after an encode.
static constexpr int kDecodeXcdShift = 2;

template <int BITS, int G, int NW>
struct RowsOut {
  static constexpr int NP = 8 / BITS;
  static constexpr int OROW = NW * G * 2;           // full-precision bytes per row and plane
  static constexpr int OPAD = OROW + 16;            // LDS row pitch (spreads the 16 rows over banks)
  static constexpr int OSLOT = 16 * NP * OPAD;      // one block's tile
  static constexpr int OCH = 16 * NP * (OROW / 16); // 16-byte chunks per tile
  static_assert(OROW % 16 == 0, "row segment of whole vectors");
  static_assert(OCH % (NW * 64) == 0, "tile chunks split evenly over the workgroup");
};

template <int BITS, int G, int R, int NW, bool IN, bool OUTL, bool INP = false>
struct RowsLayout {
  using Tl = StagedTile<BITS, G, R, NW>;
  using Ro = RowsOut<BITS, G, NW>;
  static constexpr int T = NW * 64;
  static constexpr int DPT = (Ro::OCH + T - 1) / T;           // input-tile chunks per thread
  static constexpr int SIDE = OUTL ? 16 * kSideMax * 2 : 0;    // side columns per block
  static constexpr int SPT = OUTL ? (16 * kSideMax + T - 1) / T : 0;
  static constexpr int ISLOT = Tl::SLOT + SIDE;                // staged inputs per block
  // IN && !INP: dY has tiles of its own; INP: dY is staged into the output tiles (in place)
  static constexpr size_t FIXED = 2 * (size_t)ISLOT + (IN && !INP ? 2 : 0) * (size_t)Ro::OSLOT + 2 * (size_t)Ro::OSLOT;
  static size_t bytes(int N) { return FIXED + (OUTL ? (size_t)(N / 32) * 4 + (size_t)N * 2 : 0); }
  // registers a block's prefetched inputs take per lane (drives the largest RBW)
  static constexpr int kRegsPerBlock = 4 * Tl::CPT + 1 + (IN ? 4 * DPT : 0) + SPT;
};

template <int BITS, int G, int R, int NW, int PD, bool OUTL, bool INP, class EPI, int SLN>
__global__ __launch_bounds__(NW * 64) void k_decode_rows(
    const uint8_t* __restrict__ codes, int64_t ldc, const uint16_t* __restrict__ qparams, int64_t ldq,
    const uint16_t* __restrict__ Lin, int64_t ldl, const uint16_t* __restrict__ V, int M, int N,
    const int32_t* __restrict__ oidx, int nout, const uint16_t* __restrict__ side, int64_t ldside, EPI epi,
    int RBW) {
  constexpr bool IN = EPI::kIn;
  static_assert(!INP || IN, "in-place staging is for consumers");
  static_assert(!(INP && EPI::kRot), "a rotated consumer keeps its second tensor in tiles of its own");
  using Lay = RowsLayout<BITS, G, R, NW, IN, OUTL, INP>;
  using Tl = typename Lay::Tl;
  using Ro = typename Lay::Ro;
  constexpr int NP = 8 / BITS, RT = R > 0 ? R / 16 : 1, E = G / 4, T = Lay::T;
  extern __shared__ __attribute__((aligned(16))) unsigned char sm[];
  unsigned char* ism = sm;                                   // [2][ISLOT] staged codes/qparams/L/side
  unsigned char* osm = sm + 2 * Lay::ISLOT + (IN && !INP ? 2 : 0) * Ro::OSLOT;  // [2][OSLOT] output tiles
  unsigned char* dsm = INP ? osm : sm + 2 * Lay::ISLOT;      // [2][OSLOT] input tiles (IN)
  uint32_t* colmask = reinterpret_cast<uint32_t*>(osm + 2 * Ro::OSLOT);  // OUTL: N/32 words
  int16_t* oslot = reinterpret_cast<int16_t*>(colmask + N / 32);         // OUTL: N entries
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform
  const int j = lane & 15, g = lane >> 4;
  const int units = N / (G * NP);
  const int u0 = blockIdx.y * NW, u = u0 + w;
  const int nu = min(NW, units - u0);  // units present in this workgroup
  const bool active = w < nu;
  const int vbytes = nu * G * 2;       // valid bytes of a row segment
  const int nrb = (M + 15) / 16;
  // XCD-weighted runs (the plain decode's straight-line shape, an even grid that covers the rows
  // exactly): workgroups are dealt to the 8 XCDs round robin, so with an even grid.x the odd
  // blockIdx.x are the odd XCDs, which decode about 11 % slower than the even ones right after an
  // encode (per-wave timestamps: every block of theirs, wherever its rows lie).  Each pair of
  // workgroups splits its 2 RBW blocks as RBW + XS (even) and RBW - XS (odd).
  constexpr int XS = kDecodeXcdShift;
  const bool xsplit = SLN > XS && RBW == SLN && (gridDim.x & 1) == 0 && nrb == (int)gridDim.x * RBW;
  const int xx = blockIdx.x;
  const int rb0 = xsplit ? (xx / 2) * 2 * RBW + ((xx & 1) ? RBW + XS : 0) : xx * RBW;
  if (rb0 >= nrb) return;  // whole workgroup (no barrier reached)
  const int nblk = xsplit ? ((xx & 1) ? RBW - XS : RBW + XS) : min(RBW, nrb - rb0);

  if constexpr (OUTL) {
    for (int i = tid; i < N / 32; i += T) colmask[i] = 0u;
    for (int i = tid; i < N; i += T) oslot[i] = -1;
    __syncthreads();
    for (int k = tid; k < nout; k += T) {
      const int c = oidx[k];
      if (c >= 0 && c < N) {
        atomicOr(&colmask[c >> 5], 1u << (c & 31));
        oslot[c] = (int16_t)k;
      }
    }
    // made visible by the first block's barrier
  }

  // V operands: requested right before the first blocks' inputs (below); unconditional (see
  // below), waves past the last unit load the last unit's operands
  u32x2 vop[NP][G / 16][RT];
  auto load_v = [&]() __attribute__((always_inline)) {
    if constexpr (R > 0) {
#pragma unroll
      for (int p = 0; p < NP; ++p) load_vops<G, R>(V, unit_base(p, min(u, units - 1), N, NP, G), j, g, vop[p]);
    }
  };

  struct In {
    u32x4 c[Tl::CPT];
    uint32_t ql;
    u32x4 d[IN ? Lay::DPT : 1];
    uint32_t sd[OUTL ? Lay::SPT : 1];
  };
  // Every global load and store of the block loop is issued by every lane, unconditionally:
  // a load or store under a per-lane branch makes the compiler drain all outstanding memory
  // operations (the prefetched blocks included) before the next use of any load.  Lanes whose
  // chunk lies past the workgroup's units load a clamped (valid) address and stage the value
  // where nothing reads it; their stores are dropped by the buffer range check.
  // qparams and L move as 4-byte chunks, one per thread and block: threads 0 .. QCH4 - 1 take the
  // qparam pairs (QROW / 4 per row), the next LCH4 threads the L row pieces, and any further
  // threads repeat the last chunk (the same bytes to the same LDS word).  One unconditional load
  // per thread: with a load under a per-lane branch the compiler waited for every outstanding
  // load (vmcnt(0)) inside the prefetch, so no block could start before all had arrived.
  constexpr int QCH4 = 4 * Tl::QROW, LCH4 = R > 0 ? 4 * Tl::LROW : 0;
  static_assert(QCH4 + LCH4 <= T, "one qparam / L chunk per thread");
  const int qlk = min(tid, QCH4 + LCH4 - 1);
  const bool is_q = qlk < QCH4;  // wave-uniform except in the wave holding the q / L boundary
  const int qr = qlk / (Tl::QROW / 4), qc4 = qlk % (Tl::QROW / 4);
  const int lk = max(qlk - QCH4, 0), lr = lk / (R > 0 ? Tl::LROW / 4 : 1), lc4 = lk % (R > 0 ? Tl::LROW / 4 : 1);
  // tile chunk k -> (plane, row, 16-byte column chunk)
  auto chunk = [](int k, int& p, int& r, int& c16) {
    c16 = k % (Ro::OROW / 16);
    const int pr = k / (Ro::OROW / 16);
    p = pr / 16;
    r = pr % 16;
  };
  // Addresses: a chunk's column bytes are fixed per thread; its row enters as
  // min(r, last row of the matrix - first row of the block) times the row stride, added to the
  // wave-uniform base of the block (rows past the end repeat the last row).
  const uint32_t ccol = (uint32_t)u0 * G;
  const int64_t ldc_b = ldc, ldq_b = ldq * 2, ldl_b = ldl * 2;
  const int64_t ldi_b = epi.in_ld() * 2, ldo_b = epi.out_ld() * 2;
  auto rowclamp = [&](int rb, int r) __attribute__((always_inline)) { return (uint32_t)min(r, M - 1 - rb * 16); };
  auto load = [&](In& in, int rb) __attribute__((always_inline)) {
    const unsigned char* cb0 = codes + (int64_t)rb * 16 * ldc_b;
#pragma unroll
    for (int i = 0; i < Tl::CPT; ++i) {
      const int k = tid + T * i, r = k / (Tl::CROW / 16), c16 = min(k % (Tl::CROW / 16), nu * (G / 16) - 1);
      in.c[i] = ld16_stream(cb0 + rowclamp(rb, r) * (uint32_t)ldc_b + ccol + c16 * 16);
    }
    {
      const unsigned char* qa = reinterpret_cast<const unsigned char*>(qparams) + (int64_t)rb * 16 * ldq_b +
                                rowclamp(rb, qr) * (uint32_t)ldq_b + (uint32_t)u0 * NP * 4 + min(qc4, nu * NP - 1) * 4;
      const unsigned char* la = R > 0 ? reinterpret_cast<const unsigned char*>(Lin) + (int64_t)rb * 16 * ldl_b +
                                            rowclamp(rb, lr) * (uint32_t)ldl_b + lc4 * 4
                                      : qa;
      in.ql = ld4(is_q ? qa : la);
    }
    if constexpr (IN) {
      const unsigned char* ib0 = reinterpret_cast<const unsigned char*>(epi.in_row((int64_t)rb * 16));
#pragma unroll
      for (int i = 0; i < Lay::DPT; ++i) {
        const int k = tid + T * i;
        int p, r, c16;
        chunk(k, p, r, c16);
        c16 = min(c16, vbytes / 16 - 1);
        in.d[i] = ld16_stream(ib0 + rowclamp(rb, r) * (uint32_t)ldi_b + (uint32_t)unit_base(p, u0, N, NP, G) * 2 +
                              c16 * 16);
      }
    }
    if constexpr (OUTL) {
#pragma unroll
      for (int i = 0; i < Lay::SPT; ++i) {
        const int k = tid + T * i, r = k / kSideMax, c = min(k % kSideMax, nout - 1);
        in.sd[i] = side[min(rb * 16 + r, M - 1) * ldside + c];
      }
    }
  };
  auto stage = [&](const In& in, int b) __attribute__((always_inline)) {
    unsigned char* slot = ism + (b & 1) * Lay::ISLOT;
#pragma unroll
    for (int i = 0; i < Tl::CPT; ++i) {
      const int k = tid + T * i, r = k / (Tl::CROW / 16), c16 = k % (Tl::CROW / 16);
      *reinterpret_cast<u32x4*>(slot + r * Tl::CROW + c16 * 16) = in.c[i];
    }
    *reinterpret_cast<uint32_t*>(slot + (is_q ? Tl::QOFF + qr * Tl::QROW + qc4 * 4 : Tl::LOFF + lr * Tl::LROW + lc4 * 4)) =
        in.ql;
    if constexpr (IN) {
      unsigned char* ds = dsm + (b & 1) * Ro::OSLOT;
#pragma unroll
      for (int i = 0; i < Lay::DPT; ++i) {
        const int k = tid + T * i;
        int p, r, c16;
        chunk(k, p, r, c16);
        *reinterpret_cast<u32x4*>(ds + (p * 16 + r) * Ro::OPAD + c16 * 16) = in.d[i];
      }
    }
    if constexpr (OUTL) {
      uint16_t* ss = reinterpret_cast<uint16_t*>(slot + Tl::SLOT);
#pragma unroll
      for (int i = 0; i < Lay::SPT; ++i) {
        const int k = tid + T * i;
        if (k < 16 * kSideMax && (k % kSideMax) < nout) ss[k] = (uint16_t)in.sd[i];
      }
    }
  };
  auto store_tile = [&](int rb, int b) __attribute__((always_inline)) {
    const unsigned char* os = osm + (b & 1) * Ro::OSLOT;
    unsigned char* ob0 = reinterpret_cast<unsigned char*>(epi.out_row((int64_t)rb * 16));
#pragma unroll
    for (int i = 0; i < Ro::OCH / T; ++i) {
      const int k = tid + T * i;
      int p, r, c16;
      chunk(k, p, r, c16);
      const u32x4 v = *reinterpret_cast<const u32x4*>(os + (p * 16 + r) * Ro::OPAD + c16 * 16);
      st16_pred_stream(ob0, (uint32_t)(16 * ldo_b),
                       rowclamp(rb, r) * (uint32_t)ldo_b + (uint32_t)unit_base(p, u0, N, NP, G) * 2 + c16 * 16, v,
                       c16 * 16 < vbytes);
    }
  };

  // Ring of PD prefetched blocks.  Block b + PD is requested right after block b - 1's
  // stores (a store queued behind loads waits for them), so each iteration's traffic is
  // [stores of b - 1, loads of b + PD].  With PD >= the workgroup's blocks every load is issued
  // before the first store.
  // rotated output (EPI::kRot): wave w rotates 128-column block w of the tile (plane
  // w / (NW*G/128), block w % (NW*G/128) of that plane's row segment) once every wave's unit
  // is in the tile; blocks that reach past the workgroup's units are left alone (never stored)
  constexpr int RPP = NW * G / 128;  // rotation blocks per plane of a tile row
  static_assert(!EPI::kRot || (NP * RPP == NW && G % 64 == 0), "one rotation block per wave");
  u32x4 wop[EPI::kRot ? 2 : 1][2];
  if constexpr (EPI::kRot) {
#pragma unroll
    for (int q0 = 0; q0 < 2; ++q0)
#pragma unroll
      for (int n = 0; n < 2; ++n) wop[q0][n] = wht_base_operand(j, g, q0, n != 0);
  }
  const int rot_p = w / RPP, rot_q = w % RPP;
  const bool rot_live = (rot_q + 1) * (128 / G) <= nu;  // the block's units are all present

  In in[PD];
  // Position b of the workgroup's sequence, row block rb, from ring slot k: stage it, store the
  // tile of position b - 1 (row block rb_prev), then NEXT(): whatever the caller requests with the
  // slot free (RELOAD 1: row block rb + PD if position b + PD exists; 2: always; 0: nothing), then
  // reconstruct block b into its tile.
  auto body_at = [&](auto kc, int b, int rb, int rb_prev, auto next) __attribute__((always_inline)) {
    constexpr int k = decltype(kc)::value;
    stage(in[k], b);
    lds_barrier();
    if (b > 0) store_tile(rb_prev, b - 1);
    // in place: block b + 1's dY goes into the tile just stored, so every wave's reads of it
    // must have returned first
    if constexpr (INP) lds_barrier();
    next();
    if (active) {
      const unsigned char* slot = ism + (b & 1) * Lay::ISLOT;
      u32x4 cb[G / 64];
#pragma unroll
      for (int i = 0; i < G / 64; ++i)
        cb[i] = *reinterpret_cast<const u32x4*>(slot + j * Tl::CROW + w * G + E * g + 16 * i);
      uint32_t qp[NP];
      if constexpr (NP == 2) {
        const u32x2 q = *reinterpret_cast<const u32x2*>(slot + Tl::QOFF + j * Tl::QROW + w * 8);
        qp[0] = q[0];
        qp[1] = q[1];
      } else {
        qp[0] = *reinterpret_cast<const uint32_t*>(slot + Tl::QOFF + j * Tl::QROW + w * 4);
      }
      u32x2 lop[RT];
      if constexpr (R > 0) {
#pragma unroll
        for (int t = 0; t < RT; ++t)
          lop[t] = *reinterpret_cast<const u32x2*>(slot + Tl::LOFF + j * Tl::LROW + 32 * t + 8 * g);
      }
      const unsigned char* ds = dsm + (b & 1) * Ro::OSLOT;
      unsigned char* os = osm + (b & 1) * Ro::OSLOT;
#pragma unroll
      for (int p = 0; p < NP; ++p) {
        float xh[E];
        reconstruct_plane<BITS, G, R>(cb, qp[p], p, vop[p], lop, xh);
        if constexpr (OUTL && !EPI::kRot) {  // (the rotated format: after the rotation, below)
          // the lane's outlier columns one by one (usually none or one): a select over the E
          // values per outlier, instead of a test, a table read and a select per value
          const int c0 = unit_base(p, u, N, NP, G) + E * g;  // E consecutive columns in one mask word
          uint32_t mbits = (colmask[c0 >> 5] >> (c0 & 31)) & (uint32_t)((1ull << E) - 1ull);
          const uint16_t* ss = reinterpret_cast<const uint16_t*>(slot + Tl::SLOT) + j * kSideMax;
          while (mbits != 0u) {
            const int e0 = __builtin_ctz(mbits);
            mbits &= mbits - 1u;
            const float v = f16_val(ss[oslot[c0 + e0]]);
#pragma unroll
            for (int e = 0; e < E; ++e) xh[e] = e == e0 ? v : xh[e];
          }
        }
#pragma unroll
        for (int kk = 0; kk < E / 8; ++kk) {
          const int off = (p * 16 + j) * Ro::OPAD + (w * G + E * g + 8 * kk) * 2;
          u32x4 dv = u32x4{0u, 0u, 0u, 0u};
          if constexpr (IN) dv = *reinterpret_cast<const u32x4*>(ds + off);
          *reinterpret_cast<u32x4*>(os + off) = epi.apply(xh + 8 * kk, dv);
        }
      }
    }
    if constexpr (EPI::kRot) {
      lds_barrier();  // every wave's unit of block b is in the tile
      if (rot_live) {
        const int roff = (rot_p * 16 + j) * Ro::OPAD + (128 * rot_q + 32 * g) * 2;
        // OUTL: the side columns enter after the rotation; the lane's 32 columns c0 .. c0+31 of
        // the block share one mask word
        const int c0 = unit_base(rot_p, u0, N, NP, G) + 128 * rot_q + 32 * g;
        const uint32_t mword = OUTL ? colmask[c0 >> 5] : 0u;
        const uint16_t* ss = reinterpret_cast<const uint16_t*>(ism + (b & 1) * Lay::ISLOT + Tl::SLOT) + j * kSideMax;
        auto subst = [&](int k, const float* y, float* o) __attribute__((always_inline)) {
#pragma unroll
          for (int e = 0; e < 8; ++e) o[e] = y[e];
          if constexpr (OUTL) {
            uint32_t m8 = (mword >> (8 * k)) & 0xffu;
            while (m8 != 0u) {
              const int e0 = __builtin_ctz(m8);
              m8 &= m8 - 1u;
              const float v = f16_val(ss[oslot[c0 + 8 * k + e0]]);
#pragma unroll
              for (int e = 0; e < 8; ++e) o[e] = e == e0 ? v : o[e];
            }
          }
        };
        if constexpr (IN) {
          // the consumer's second tensor sits at the same place in the input tile
          const unsigned char* rd = dsm + (b & 1) * Ro::OSLOT + roff;
          wht128_lds_map(osm + (b & 1) * Ro::OSLOT + roff, wop, [&](int k, const float* y) {
            float o[8];
            subst(k, y, o);
            return epi.rot_apply(o, *reinterpret_cast<const u32x4*>(rd + 16 * k));
          });
        } else if constexpr (OUTL) {
          wht128_lds_map(osm + (b & 1) * Ro::OSLOT + roff, wop, [&](int k, const float* y) {
            float o[8];
            subst(k, y, o);
            return pack8(o);
          });
        } else {
          wht128_lds(osm + (b & 1) * Ro::OSLOT + roff, wop);
        }
      }
    }
  };
  auto body = [&](auto kc, int b, auto reload) __attribute__((always_inline)) {
    constexpr int k = decltype(kc)::value;
    const int rb = rb0 + b;
    body_at(kc, b, rb, rb - 1, [&]() {
      if constexpr (decltype(reload)::value != 0) {
        if (decltype(reload)::value == 2 || b + PD < nblk) {
          __builtin_amdgcn_sched_barrier(0);
          load(in[k], rb + PD);
          __builtin_amdgcn_sched_barrier(0);
        }
      }
    });
  };
  // Straight-line code for the workgroup's usual block counts (SLN, or SLN -+ XS under the XCD
  // split): every block without conditions, so that each block waits only for its own loads (a
  // counted vmcnt).  Under the loop below (or loads under conditions) the compiler merges the
  // paths' pending counts and each block waited for every outstanding memory operation, the
  // previous block's stores included.  (The V operands first: loads retire in issue order, so
  // block 0 waits for them and its own inputs, not for the later blocks'.)
  auto straight = [&](auto sln) __attribute__((always_inline)) {
    constexpr int SL = decltype(sln)::value;
    load_v();
    __builtin_amdgcn_sched_barrier(0);
    static_for<0, (PD < SL ? PD : SL)>([&](auto kc) { load(in[decltype(kc)::value], rb0 + decltype(kc)::value); });
    __builtin_amdgcn_sched_barrier(0);
    static_for<0, SL>([&](auto bc) {
      constexpr int b = decltype(bc)::value;
      body(std::integral_constant<int, b % PD>{}, b, std::integral_constant<int, (b + PD < SL) ? 2 : 0>{});
    });
  };
  if (SLN > 0 && nblk == SLN) {
    straight(std::integral_constant<int, SLN>{});
  } else if (SLN > XS && nblk == SLN - XS) {
    straight(std::integral_constant<int, (SLN > XS ? SLN - XS : 1)>{});
  } else if (SLN > XS && nblk == SLN + XS) {
    straight(std::integral_constant<int, SLN + XS>{});
  } else {
    load_v();
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int b = 0; b < PD; ++b)
      if (b < nblk) load(in[b], rb0 + b);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll 1
    for (int bb = 0; bb < nblk; bb += PD)
      static_for<0, PD>([&](auto kc) {
        if (bb + decltype(kc)::value < nblk) body(kc, bb + decltype(kc)::value, std::integral_constant<int, 1>{});
      });
  }
  lds_barrier();
  store_tile(rb0 + nblk - 1, nblk - 1);
}

// ------------------------------------------------------------------ host side
// Waves per workgroup for k_decode_rows: NW * G = 512 columns, so each row segment is 1 KB (one
// 16-byte vector per lane) and the tiles plus two input slots fit in LDS.
template <int BITS, int G>
constexpr int rows_nw() { return G * (8 / BITS) <= 128 ? 8 : 4; }

// One workgroup per CU: the workgroups of a unit group split its row blocks into runs of RBW
// consecutive blocks, RBW being the smallest run that keeps the grid within one round.  The ring
// holds up to 16 blocks of staged inputs within a register budget of about 180 VGPRs (rank 32:
// 160, its V operands are twice as large; consumers: 100, their epilogue and the streamed loop
// need the rest).
// Row blocks per workgroup that the plain decode runs as straight-line code (other counts, and
// the consumers, take the kernel's loop): the count the grid below gives at 16384 rows and 4096
// columns.  (Straight-line code for every instantiation would multiply the compile time.)
constexpr int kDecodeRun = 16;

template <int BITS, int G, int R, bool OUTL, class EPI>
static int decode_rows_launch(const lrq_tensors* t, hipStream_t s, const EPI& epi) {
  // a rotated consumer of int8/g128 takes 4 units per workgroup: with 8 its dY and output tiles
  // (four of 32 KB) and the staged inputs do not fit in LDS
  constexpr int NW = (EPI::kIn && EPI::kRot && BITS == 8 && G == 128) ? 4 : rows_nw<BITS, G>();
  // consumers of 128-column groups stage dY in place (separate tiles would not fit in LDS; a
  // rotated consumer cannot, and is refused by the LDS check below)
  constexpr bool INP = EPI::kIn && G == 128 && !EPI::kRot;
  using Lay = RowsLayout<BITS, G, R, NW, EPI::kIn, OUTL, INP>;
  constexpr int kBudget = EPI::kIn ? 100 : EPI::kRot ? 150 : R == 32 ? 160 : 180;
  constexpr int kFit = kBudget / Lay::kRegsPerBlock;
  // (a rotated consumer at rank 32, or with side columns, also holds the rotation operands and
  // the substitution's state: two blocks in flight; the rotated decode with side columns: four)
  constexpr int PD = (EPI::kIn && EPI::kRot && (R == 32 || OUTL)) ? 2
                     : (EPI::kRot && OUTL)                           ? 4
                     : kFit >= 16                                    ? 16
                     : kFit >= 8                                     ? 8
                     : kFit >= 4                                     ? 4
                                                                     : 2;
  const int M = (int)t->rows, N = (int)t->hidden;
  const int units = N / (G * (8 / BITS));
  const int64_t ug = (units + NW - 1) / NW, nrb = (M + 15) / 16, cus = cu_count();
  const int64_t per = std::max<int64_t>(1, cus / ug);  // workgroups per unit group
  const int rbw = (int)((nrb + per - 1) / per);
  const size_t shm = Lay::bytes(N);
  if (shm > 160 * 1024) return LRQ_ERR_UNSUPPORTED;
  constexpr int SLN = (!EPI::kIn && !EPI::kRot && !OUTL) ? kDecodeRun : 0;
  auto kern = k_decode_rows<BITS, G, R, NW, PD, OUTL, INP, EPI, SLN>;
  if (shm > 64 * 1024) (void)hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)shm);
  LRQ_TRY(launch(kern, dim3((unsigned)((nrb + rbw - 1) / rbw), (unsigned)ug), dim3(NW * 64), shm, s,
                     (const uint8_t*)t->codes, t->ld_codes, (const uint16_t*)t->qparams, t->ld_qp,
                     (const uint16_t*)t->L, t->ld_L, (const uint16_t*)t->V, M, N, t->outlier_idx, (int)t->n_outlier,
                     (const uint16_t*)t->side, t->ld_side, epi, rbw));
  return LRQ_OK;
}

template <int BITS, int G, int R, int RBW, class EPI>
static int decode_launch_rbw(const lrq_tensors* t, hipStream_t s, const EPI& epi) {
  constexpr int NP = 8 / BITS, NW = 8, PD = RBW;  // every load before the first store
  const int M = (int)t->rows, N = (int)t->hidden;
  const int units = N / (G * NP);
  const int nrb = (M + 15) / 16;
  dim3 grid((nrb + RBW - 1) / RBW, (units + NW - 1) / NW);
  if (t->n_outlier > 0) {
    const size_t shm = (size_t)(N / 32) * 4 + (size_t)N * 2;
    LRQ_TRY(launch((k_decode<BITS, G, R, true, NW, RBW, PD, EPI>), grid, dim3(NW * 64), shm, s,
                       (const uint8_t*)t->codes, t->ld_codes, (const uint16_t*)t->qparams, t->ld_qp,
                       (const uint16_t*)t->L, t->ld_L, (const uint16_t*)t->V, M, N, t->outlier_idx, t->n_outlier,
                       (const uint16_t*)t->side, t->ld_side, epi));
  } else {
    const size_t shm = 2 * (size_t)StagedTile<BITS, G, R, NW>::SLOT;
    LRQ_TRY(launch((k_decode_staged<BITS, G, R, NW, RBW, EPI>), grid, dim3(NW * 64), shm, s,
                       (const uint8_t*)t->codes, t->ld_codes, (const uint16_t*)t->qparams, t->ld_qp,
                       (const uint16_t*)t->L, t->ld_L, (const uint16_t*)t->V, M, N, epi));
  }
  return LRQ_OK;
}

// 8 row blocks per wave (4 when the consumer also streams a second tensor in) when that
// still leaves >= 512 workgroups (2 per CU), else 2.
template <int BITS, int G, int R, class EPI>
static int decode_launch(const lrq_tensors* t, hipStream_t s, const EPI& epi) {
  constexpr int NP = 8 / BITS, NW = 8, BIG = EPI::kIn ? 4 : 8;
  // The row kernel addresses a block's rows by 32-bit offsets: 16 rows of every operand must
  // stay below 2^31 bytes (always true for real hidden sizes; the others take the tile kernels).
  bool off32 = true;
  for (int64_t ldb : {t->ld_codes, 2 * t->ld_qp, 2 * t->ld_L, 2 * epi.in_ld(), 2 * epi.out_ld()})
    off32 = off32 && 16 * ldb < ((int64_t)1 << 31);
  if (off32 && t->n_outlier == 0) return decode_rows_launch<BITS, G, R, false>(t, s, epi);
  if (off32 && t->n_outlier <= kSideMax) {
    // the row kernel's tiles, side slots and outlier tables may not fit in LDS (a consumer at
    // rank > 0): then the tile kernel below
    const int st = decode_rows_launch<BITS, G, R, true>(t, s, epi);
    if (st != LRQ_ERR_UNSUPPORTED) return st;
  }
  const int64_t units = t->hidden / (G * NP), nrb = (t->rows + 15) / 16;
  const int64_t wgs = ((nrb + BIG - 1) / BIG) * ((units + NW - 1) / NW);
  if (wgs >= 512) return decode_launch_rbw<BITS, G, R, BIG>(t, s, epi);
  return decode_launch_rbw<BITS, G, R, 2>(t, s, epi);
}

template <class EPI>
static int decode_dispatch(const lrq_tensors* t, hipStream_t s, const EPI& epi) {
  if (t->flags & LRQ_FLAG_HADAMARD) return LRQ_ERR_UNSUPPORTED;
  switch (format_key(t->bits, t->group, t->rank)) {
    case format_key(4, 64, 0): return decode_launch<4, 64, 0>(t, s, epi);
    case format_key(4, 64, 16): return decode_launch<4, 64, 16>(t, s, epi);
    case format_key(4, 64, 32): return decode_launch<4, 64, 32>(t, s, epi);
    case format_key(4, 128, 0): return decode_launch<4, 128, 0>(t, s, epi);
    case format_key(4, 128, 16): return decode_launch<4, 128, 16>(t, s, epi);
    case format_key(8, 64, 0): return decode_launch<8, 64, 0>(t, s, epi);
    case format_key(8, 64, 16): return decode_launch<8, 64, 16>(t, s, epi);
    case format_key(8, 128, 0): return decode_launch<8, 128, 0>(t, s, epi);
    case format_key(8, 128, 16): return decode_launch<8, 128, 16>(t, s, epi);
    default: return LRQ_ERR_UNSUPPORTED;
  }
}

static int check_io(const lrq_tensors* t, const void* in, int64_t ldin, const void* out, int64_t ldout,
                    bool need_in) {
  int st = validate_tensors(t);
  if (st) return st;
  if (need_in) {
    st = validate_rows16(in, ldin, t->hidden);
    if (st) return st;
  }
  return validate_rows16(out, ldout, t->hidden);
}

}  // namespace lrq

using namespace lrq;

namespace lrq {
// Rotated format, fused: the row kernel undoes the rotation on its LDS output tile, then writes
// the side columns over it.  Formats with one 128-column rotation block per wave (int4/g64,
// int8/g128), up to kSideMax outlier channels, and planes that are whole rotation blocks;
// returns 0 for the others.
template <int BITS, int G, int R>
static int decode_rot_fused(const lrq_tensors* t, hipStream_t s, uint16_t* out, int64_t ldo, int* status) {
  if constexpr (!((BITS == 4 && G == 64) || (BITS == 8 && G == 128))) {
    return 0;
  } else {
    const int64_t plane = t->hidden / (8 / BITS);
    if (t->n_outlier > kSideMax || plane % 128 != 0) return 0;
    for (int64_t ldb : {t->ld_codes, 2 * t->ld_qp, 2 * t->ld_L, 2 * ldo, 2 * t->ld_side})
      if (16 * ldb >= ((int64_t)1 << 31)) return 0;
    lrq_tensors plain = *t;
    plain.flags &= ~LRQ_FLAG_HADAMARD;
    EpiStoreRot epi;
    epi.out = out;
    epi.ld = ldo;
    const int st = t->n_outlier > 0 ? decode_rows_launch<BITS, G, R, true>(&plain, s, epi)
                                    : decode_rows_launch<BITS, G, R, false>(&plain, s, epi);
    if (st == LRQ_ERR_UNSUPPORTED) return 0;  // its tiles do not fit in LDS
    *status = st;
    return 1;
  }
}

// out[r, idx[k]] = bf16(side[r, k]) (indices outside [0, N) skipped): the side columns of the
// rotated format, written after the separate rotation pass.
__global__ __launch_bounds__(256) void k_scatter_side(const uint16_t* __restrict__ side, int64_t ldside, int M, int N,
                                                      const int32_t* __restrict__ oidx, int nout,
                                                      uint16_t* __restrict__ out, int64_t ldo) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (int64_t)M * nout) return;
  const int64_t r = i / nout;
  const int k = (int)(i - r * nout);
  const int c = oidx[k];
  if (c < 0 || c >= N) return;
  out[r * ldo + c] = (uint16_t)pack_bf16x2(f16_val(side[r * ldside + k]), 0.f);
}

// Rotated format with a consumer, fused into the row kernel (EpiRot): int4/g64 (int8/g128's
// row kernel has no LDS left for the consumer's own tiles), up to kSideMax outlier channels,
// planes of whole rotation blocks; returns 0 for the others.
template <int BITS, int G, int R, class EPI>
static int consumer_rot_fused(const lrq_tensors* t, hipStream_t s, const EPI& inner, int* status) {
  if constexpr (!((BITS == 4 && G == 64) || (BITS == 8 && G == 128))) {
    return 0;
  } else {
    const int64_t plane = t->hidden / (8 / BITS);
    if (t->n_outlier > kSideMax || plane % 128 != 0) return 0;
    for (int64_t ldb : {t->ld_codes, 2 * t->ld_qp, 2 * t->ld_L, 2 * inner.in_ld(), 2 * inner.out_ld(), 2 * t->ld_side})
      if (16 * ldb >= ((int64_t)1 << 31)) return 0;
    lrq_tensors plain = *t;
    plain.flags &= ~LRQ_FLAG_HADAMARD;
    EpiRot<EPI> epi;
    static_cast<EPI&>(epi) = inner;
    const int st = t->n_outlier > 0 ? decode_rows_launch<BITS, G, R, true>(&plain, s, epi)
                                    : decode_rows_launch<BITS, G, R, false>(&plain, s, epi);
    if (st == LRQ_ERR_UNSUPPORTED) return 0;
    *status = st;
    return 1;
  }
}

template <class EPI>
static int consumer_rot(const lrq_tensors* t, hipStream_t s, const EPI& inner, int* status) {
  switch (format_key(t->bits, t->group, t->rank)) {
    case format_key(4, 64, 0): return consumer_rot_fused<4, 64, 0>(t, s, inner, status);
    case format_key(4, 64, 16): return consumer_rot_fused<4, 64, 16>(t, s, inner, status);
    case format_key(4, 64, 32): return consumer_rot_fused<4, 64, 32>(t, s, inner, status);
    case format_key(8, 128, 0): return consumer_rot_fused<8, 128, 0>(t, s, inner, status);
    case format_key(8, 128, 16): return consumer_rot_fused<8, 128, 16>(t, s, inner, status);
    default: return 0;
  }
}

static int decode_rot(const lrq_tensors* t, hipStream_t s, uint16_t* out, int64_t ldo, int* status) {
  switch (format_key(t->bits, t->group, t->rank)) {
    case format_key(4, 64, 0): return decode_rot_fused<4, 64, 0>(t, s, out, ldo, status);
    case format_key(4, 64, 16): return decode_rot_fused<4, 64, 16>(t, s, out, ldo, status);
    case format_key(4, 64, 32): return decode_rot_fused<4, 64, 32>(t, s, out, ldo, status);
    case format_key(8, 128, 0): return decode_rot_fused<8, 128, 0>(t, s, out, ldo, status);
    case format_key(8, 128, 16): return decode_rot_fused<8, 128, 16>(t, s, out, ldo, status);
    default: return 0;
  }
}
}  // namespace lrq

extern "C" int lrq_decode(const lrq_tensors* t, void* out, int64_t ldo, void* stream) {
  int st = check_io(t, nullptr, 0, out, ldo, false);
  if (st) return st;
  if (t->rows == 0) return LRQ_OK;
  if (t->flags & LRQ_FLAG_HADAMARD) {
    if (decode_rot(t, (hipStream_t)stream, (uint16_t*)out, ldo, &st)) return st;
    // otherwise decode, undo the rotation in place (the rotation is its own inverse), then
    // write the side columns
    lrq_tensors plain = *t;
    plain.flags &= ~LRQ_FLAG_HADAMARD;
    plain.n_outlier = 0;
    LRQ_TRY(decode_dispatch(&plain, (hipStream_t)stream, EpiStore{(uint16_t*)out, ldo}));
    LRQ_TRY(lrq_wht128(out, ldo, t->rows, t->hidden, out, ldo, stream));
    if (t->n_outlier == 0) return LRQ_OK;
    const int64_t n = t->rows * t->n_outlier;
    LRQ_TRY(launch(k_scatter_side, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                   (const uint16_t*)t->side, t->ld_side, (int)t->rows, (int)t->hidden, t->outlier_idx,
                   (int)t->n_outlier, (uint16_t*)out, ldo));
    return LRQ_OK;
  }
  return decode_dispatch(t, (hipStream_t)stream, EpiStore{(uint16_t*)out, ldo});
}

namespace lrq {
// The elementwise consumers (op as lrq_dense_elementwise numbers them).  The rotated format goes
// to the fused row kernel where it can, else decode into `out` (rotation undone) and the dense
// op in place over it: two kernels, no scratch.  The second form needs rows of exactly `hidden`
// elements in both tensors (the dense kernel is flat) and `out` distinct from `in` (the decode
// would overwrite `in` before the op reads it).
template <class EPI>
static int consumer(const lrq_tensors* t, const void* in, int64_t ldin, void* out, int64_t ldo, int op,
                    void* stream) {
  int st = check_io(t, in, ldin, out, ldo, true);
  if (st) return st;
  if (t->rows == 0) return LRQ_OK;
  const EPI epi{(const uint16_t*)in, ldin, (uint16_t*)out, ldo};
  if (!(t->flags & LRQ_FLAG_HADAMARD)) return decode_dispatch(t, (hipStream_t)stream, epi);
  if (consumer_rot(t, (hipStream_t)stream, epi, &st)) return st;
  if (ldin != t->hidden || ldo != t->hidden || in == out) return LRQ_ERR_UNSUPPORTED;
  LRQ_TRY(lrq_decode(t, out, ldo, stream));
  return lrq_dense_elementwise(op, out, in, out, t->rows * t->hidden, stream);
}
}  // namespace lrq

extern "C" int lrq_silu_bwd(const lrq_tensors* t, const void* dy, int64_t lddy, void* dx, int64_t lddx,
                            void* stream) {
  return consumer<EpiSilu>(t, dy, lddy, dx, lddx, 0, stream);
}

extern "C" int lrq_gelu_bwd(const lrq_tensors* t, const void* dy, int64_t lddy, void* dx, int64_t lddx,
                            void* stream) {
  return consumer<EpiGelu>(t, dy, lddy, dx, lddx, 1, stream);
}

extern "C" int lrq_mul(const lrq_tensors* t, const void* y, int64_t ldy, void* out, int64_t ldo, void* stream) {
  return consumer<EpiMul>(t, y, ldy, out, ldo, 2, stream);
}
