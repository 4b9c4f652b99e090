// Both LoRA factor-gradient products of the compressed activation in one pass over its codes:
// xa = x_hat A (for dB = (x A)^T dy) and da = x_hat^T g (dA, g = dy B^T), the two products of
// compute_lora_gradient (low_rank_system_profile_forward.py:14-18) that read the saved x.
//
// x_hat = bf16(decode) is rebuilt once per 16 x 16 tile, in the layout of the transposed product
// (as in k_dequant_gemm_t: lane (j, g) holds rows 4g .. 4g+3 of one column, the low-rank term
// added on MFMA with the dequantised value as accumulator input), and used three times:
//   da  += g^T * x_hat            (g's rows transposed once per block by an identity MFMA)
//   y    = x_hat^T * I            (identity MFMA: the tile transposed into the other layout,
//                                  lane (row, g) holding 4 columns; exact)
//   xa  += A^T * y                (A's tile columns as resident A operands)
// so the codes, qparams and L are read once for both products.  Geometry (int4 / g64 / rank 16,
// n = 16): workgroup (cg, rg) covers the 4 units 4 cg .. 4 cg + 3 (512 columns) and row blocks
// rg * bpg .. + bpg - 1; wave w = (wc, wr), wc = w % 4 its unit, wr = w / 4 its row phase, walks
// the blocks rg * bpg + wr + 2 i.  da is summed over the two row phases in LDS and leaves as one
// fp32 partial per row group; xa is summed over the four units of each block in LDS and leaves as
// one fp32 partial per column group; k_lora_sum adds the partials in a fixed order (deterministic).
#include <algorithm>

#include "lrq_common.h"
#include "lrq_host.h"

namespace lrq {

struct LoraGeo {
  static constexpr int BITS = 4, G = 64, NP = 2, UPW = 4, RPH = 2, NW = UPW * RPH;
  static constexpr int BPL = G / 16, TT = BPL;  // code bytes per lane and row = tiles per plane
  static constexpr int NBW_MAX = 16;            // most blocks per wave (register accumulators)
};

template <int NBW>
__global__ __launch_bounds__(512) void k_lora_grads(
    const uint8_t* __restrict__ codes, int64_t ldc, const uint16_t* __restrict__ qparams, int64_t ldq,
    const uint16_t* __restrict__ Lin, int64_t ldl, const uint16_t* __restrict__ V, int M, int N,
    const uint16_t* __restrict__ A, int64_t lda, const uint16_t* __restrict__ gm, int64_t ldg,
    float* __restrict__ xa_part, float* __restrict__ da_part, int bpg, int ncg) {
  using Ge = LoraGeo;
  constexpr int NP = Ge::NP, G = Ge::G, BPL = Ge::BPL, TT = Ge::TT, PD = 2;
  constexpr int XR = NBW < 4 ? NBW : 4;  // blocks per round of the xa reduction
  __shared__ f32x4 red[Ge::UPW * NP * TT > Ge::RPH * XR * Ge::UPW ? Ge::UPW * NP * TT : Ge::RPH * XR * Ge::UPW][64];
  const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int j = lane & 15, g = lane >> 4;
  const int wc = w & 3, wr = w >> 2;
  // (the divisions run on the vector unit: readfirstlane brings the uniform results back to
  // scalar registers, so that all block addressing below stays scalar)
  // the column groups of one row group on one XCD: they read the same L and g rows
  const int tile = xcd_tile(blockIdx.x, gridDim.x);
  const int cgi = __builtin_amdgcn_readfirstlane(tile % ncg);
  const int rgi = __builtin_amdgcn_readfirstlane(tile / ncg);
  const int nrb = (M + 15) / 16;
  const int rb_lo = rgi * bpg, rb_hi = min(rb_lo + bpg, nrb);  // the host gives every row group a block
  const int u = __builtin_amdgcn_readfirstlane(cgi * Ge::UPW + wc);
  const u32x2 ident = identity_bop(j, g);

  // reconstruction operands: lane (j, g) holds V[column c(j, p, t)][ranks 4g ..], c(m, p, t) =
  // p N/2 + u G + BPL m + t; xa operands: lane (k = j, g) holds A[c(4g + e, p, t)][k], e < 4
  u32x2 vop[NP][TT], aop[NP][TT];
#pragma unroll
  for (int p = 0; p < NP; ++p)
#pragma unroll
    for (int t = 0; t < TT; ++t) {
      const int64_t cb = (int64_t)p * (N / NP) + (int64_t)u * G + t;
      vop[p][t] = ld8(V + (cb + BPL * j) * 16 + 4 * g);
      uint32_t h[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) h[e] = A[(cb + BPL * (4 * g + e)) * lda + j];
      aop[p][t] = u32x2{h[0] | (h[1] << 16), h[2] | (h[3] << 16)};
    }
  f32x4 acc[NP][TT], accx[NBW];
#pragma unroll
  for (int p = 0; p < NP; ++p)
#pragma unroll
    for (int t = 0; t < TT; ++t) acc[p][t] = zero4();
#pragma unroll
  for (int i = 0; i < NBW; ++i) accx[i] = zero4();

  struct Blk {
    uint32_t cw[4];      // rows 4g + v: code bytes BPL j .. of the unit
    uint32_t qp[4][NP];  // rows 4g + v: (scale, zero) of each plane of the unit
    u32x2 lop;           // row j: L ranks 4g ..
    u32x2 gop;           // row j: g columns 4g ..
  };
  // 32-bit lane offsets from each block's wave-uniform bases; rows past the end repeat the last
  // row (min on the offsets against lim * ld, lim the block's last present row, at most 15: with
  // row strides below 2^24 bytes, checked by the launch, every offset stays below 2^28)
  const uint32_t ldc1 = (uint32_t)ldc, ldq2 = (uint32_t)ldq * 2, ldl2 = (uint32_t)ldl * 2, ldg2 = (uint32_t)ldg * 2;
  uint32_t coff[4], qoff[4];
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    coff[v] = (uint32_t)(4 * g + v) * ldc1;
    qoff[v] = (uint32_t)(4 * g + v) * ldq2;
  }
  const uint32_t loff = (uint32_t)j * ldl2, goff = (uint32_t)j * ldg2;
  const uint32_t cl = (uint32_t)(BPL * j), ql = (uint32_t)(u * NP * 4), rl = (uint32_t)(8 * g);
  auto load = [&](int rb, Blk& d) {
    const int r0 = rb * 16;
    const uint32_t lim = (uint32_t)min(M - 1 - r0, 15);
    const uint8_t* cbase = codes + (int64_t)r0 * ldc + u * G;
    const uint8_t* qbase = reinterpret_cast<const uint8_t*>(qparams + (int64_t)r0 * ldq);
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      d.cw[v] = ld4(cbase + (min(coff[v], lim * ldc1) + cl));
      const u32x2 q = ld8(qbase + (min(qoff[v], lim * ldq2) + ql));
      d.qp[v][0] = q[0];
      d.qp[v][1] = q[1];
    }
    d.lop = ld8(reinterpret_cast<const uint8_t*>(Lin + (int64_t)r0 * ldl) + (min(loff, lim * ldl2) + rl));
    d.gop = ld8(reinterpret_cast<const uint8_t*>(gm + (int64_t)r0 * ldg) + (min(goff, lim * ldg2) + rl));
  };
  auto process = [&](const Blk& cur, int rb, bool blive, f32x4& ax) {
    const bool live = blive && rb * 16 + j < M;  // g rows past M (or of a block past the wave's) add nothing
    const f32x4 d = mfma_16x16x16(live ? cur.gop : u32x2{0u, 0u}, ident, zero4());  // lane (j, g): g[4g + v][j]
    const u32x2 a2 = u32x2{pack_bf16x2_exact(d[0], d[1]), pack_bf16x2_exact(d[2], d[3])};
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      float sf[4], zf[4];
      uint32_t wq[4];  // row 4g + v: plane p's codes of tiles 0 .. 3, one per byte
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        sf[v] = f16_val(cur.qp[v][p] & 0xffffu);
        zf[v] = f16_val(cur.qp[v][p] >> 16);
        wq[v] = (cur.cw[v] >> (4 * p)) & 0x0f0f0f0fu;
      }
      // the plane's four tiles step by step, so that each step's MFMAs cover each other's latency
      f32x4 x[TT], y[TT];
      u32x2 xb[TT];
#pragma unroll
      for (int t = 0; t < TT; ++t)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const float q = t == 0 ? ubyte_f32<0>(wq[v]) : t == 1 ? ubyte_f32<1>(wq[v]) : t == 2 ? ubyte_f32<2>(wq[v])
                                                                                             : ubyte_f32<3>(wq[v]);
          x[t][v] = __builtin_fmaf(q, sf[v], zf[v]);
        }
#pragma unroll
      for (int t = 0; t < TT; ++t) x[t] = mfma_16x16x16(cur.lop, vop[p][t], x[t]);  // + (L V^T)[4g + v][col], rounded once
#pragma unroll
      for (int t = 0; t < TT; ++t) xb[t] = u32x2{pack_bf16x2(x[t][0], x[t][1]), pack_bf16x2(x[t][2], x[t][3])};  // x_hat
#pragma unroll
      for (int t = 0; t < TT; ++t) {
        y[t] = mfma_16x16x16(xb[t], ident, zero4());  // lane (row, g): x_hat[row][c(4g + v)]
        acc[p][t] = mfma_16x16x16(a2, xb[t], acc[p][t]);
      }
#pragma unroll
      for (int t = 0; t < TT; ++t)
        ax = mfma_16x16x16(aop[p][t], u32x2{pack_bf16x2_exact(y[t][0], y[t][1]), pack_bf16x2_exact(y[t][2], y[t][3])}, ax);
    }
  };

  // The wave's blocks rb_lo + wr + 2 i, i < NBW, as straight-line code (static accumulator and
  // slot indices); blocks past the wave's last are computed with a zero g and not stored.
  const int nbw = rb_lo + wr < rb_hi ? (rb_hi - rb_lo - wr + 1) / 2 : 0;
  const int last = rb_hi - 1;
  {
    Blk ring[PD];
#pragma unroll
    for (int sl = 0; sl < PD && sl < NBW; ++sl) load(min(rb_lo + wr + 2 * sl, last), ring[sl]);
    __builtin_amdgcn_sched_barrier(0);
    static_for<0, NBW>([&](auto ic) {
      constexpr int i = decltype(ic)::value;
      const int rb = rb_lo + wr + 2 * i;
      process(ring[i % PD], rb, i < nbw, accx[i]);
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (i + PD < NBW) load(min(rb + 2 * PD, last), ring[i % PD]);
      __builtin_amdgcn_sched_barrier(0);
    });
  }

  // da: the two row phases of each unit summed in order, one partial per row group:
  // acc[p][t] in lane (j, g), component v: column c(j, p, t), k = 4g + v
  if (wr == 1) {
#pragma unroll
    for (int p = 0; p < NP; ++p)
#pragma unroll
      for (int t = 0; t < TT; ++t) red[(wc * NP + p) * TT + t][lane] = acc[p][t];
  }
  __syncthreads();
  if (wr == 0) {
#pragma unroll
    for (int p = 0; p < NP; ++p)
#pragma unroll
      for (int t = 0; t < TT; ++t) {
        const f32x4 o = red[(wc * NP + p) * TT + t][lane];
        f32x4 s = acc[p][t];
        s[0] += o[0];
        s[1] += o[1];
        s[2] += o[2];
        s[3] += o[3];
        const int64_t col = (int64_t)p * (N / NP) + (int64_t)u * G + BPL * j + t;
        *reinterpret_cast<f32x4*>(da_part + ((int64_t)rgi * N + col) * 16 + 4 * g) = s;
      }
  }
  __syncthreads();

  // xa: rounds of XR blocks per row phase; wave (wr', ii) = (w / 4, w % 4) sums block ii of the
  // round of phase wr' over the four units in order: lane (row j, g) holds xa[row][4g + v]
#pragma unroll
  for (int r0 = 0; r0 < NBW; r0 += XR) {
#pragma unroll
    for (int ii = 0; ii < XR; ++ii) red[(wr * XR + ii) * Ge::UPW + wc][lane] = accx[r0 + ii];
    __syncthreads();
    const int pr = w >> 2, ii = w & 3;
    if (ii < XR && r0 + ii < (rb_lo + pr < rb_hi ? (rb_hi - rb_lo - pr + 1) / 2 : 0)) {
      f32x4 s = red[(pr * XR + ii) * Ge::UPW][lane];
#pragma unroll
      for (int c = 1; c < Ge::UPW; ++c) {
        const f32x4 o = red[(pr * XR + ii) * Ge::UPW + c][lane];
        s[0] += o[0];
        s[1] += o[1];
        s[2] += o[2];
        s[3] += o[3];
      }
      const int row = (rb_lo + pr + 2 * (r0 + ii)) * 16 + j;
      if (row < M) *reinterpret_cast<f32x4*>(xa_part + ((int64_t)cgi * M + row) * 16 + 4 * g) = s;
    }
    __syncthreads();
  }
}

// xa[row][k] = sum over the ncg column-group partials, da[col][k] = sum over the nrg row-group
// partials, each in partial order; four outputs per thread.
__global__ __launch_bounds__(256) void k_lora_sum(const float* __restrict__ xa_part, int ncg, int M,
                                                  void* __restrict__ xa, int64_t ldxa, int xa_f32,
                                                  const float* __restrict__ da_part, int nrg, int N,
                                                  void* __restrict__ da, int64_t ldda, int da_f32) {
  const int64_t q = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t nx = (int64_t)M * 4, nd = (int64_t)N * 4;
  const float* src;
  int np;
  int64_t stride, r, ld;
  void* out;
  int f32;
  if (q < nx) {
    src = xa_part, np = ncg, stride = (int64_t)M * 16, r = q >> 2, out = xa, ld = ldxa, f32 = xa_f32;
  } else if (q < nx + nd) {
    src = da_part, np = nrg, stride = (int64_t)N * 16, r = (q - nx) >> 2, out = da, ld = ldda, f32 = da_f32;
  } else {
    return;
  }
  const int k4 = (int)(q & 3) * 4;
  const float* p = src + r * 16 + k4;
  f32x4 s = np > 0 ? *reinterpret_cast<const f32x4*>(p) : zero4();  // no partials (no rows): zeros
  // the partials in chunks of 8: a chunk's loads go out together, then are added in order
  for (int i0 = 1; i0 < np; i0 += 8) {
    f32x4 o[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] = i0 + i < np ? *reinterpret_cast<const f32x4*>(p + (i0 + i) * stride) : zero4();
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      if (i0 + i < np) {
        s[0] += o[i][0];
        s[1] += o[i][1];
        s[2] += o[i][2];
        s[3] += o[i][3];
      }
    }
  }
  if (f32) {
    *reinterpret_cast<f32x4*>(reinterpret_cast<float*>(out) + r * ld + k4) = s;
  } else {
    *reinterpret_cast<u32x2*>(reinterpret_cast<uint16_t*>(out) + r * ld + k4) =
        u32x2{pack_bf16x2(s[0], s[1]), pack_bf16x2(s[2], s[3])};
  }
}

struct LoraPlan {
  int ncg = 0, nrg = 0, bpg = 0, nbw = 0;
  int64_t xa_bytes = 0, ws_bytes = 0;
};
// Column groups of 4 units; row groups of bpg blocks, about 256 workgroups, at most 2 NBW_MAX
// blocks per group, every group non-empty.
static int lora_plan(const lrq_tensors* t, int n_out, LoraPlan& pl) {
  if (t->bits != 4 || t->group != 64 || t->rank != 16 || t->flags != 0 || t->n_outlier != 0) return LRQ_ERR_UNSUPPORTED;
  if (n_out != 16) return LRQ_ERR_UNSUPPORTED;
  const int64_t units = t->hidden / 128;
  if (units % LoraGeo::UPW != 0) return LRQ_ERR_UNSUPPORTED;
  constexpr int64_t kLim = int64_t(1) << 24;  // 32-bit lane offsets of 16 rows
  if (t->ld_codes >= kLim || t->ld_qp * 2 >= kLim || t->ld_L * 2 >= kLim) return LRQ_ERR_UNSUPPORTED;
  pl.ncg = (int)(units / LoraGeo::UPW);
  const int64_t nrb = (t->rows + 15) / 16;
  if (nrb == 0) return LRQ_OK;
  const int64_t want = std::max<int64_t>(1, 256 / pl.ncg);
  int64_t bpg = std::min<int64_t>((nrb + want - 1) / want, 2 * LoraGeo::NBW_MAX);
  bpg = std::max<int64_t>(bpg, 1);
  pl.bpg = (int)bpg;
  pl.nrg = (int)((nrb + bpg - 1) / bpg);
  const int half = (int)((bpg + 1) / 2);
  pl.nbw = half <= 1 ? 1 : half <= 2 ? 2 : half <= 4 ? 4 : half <= 8 ? 8 : 16;
  pl.xa_bytes = (int64_t)pl.ncg * t->rows * 16 * 4;
  pl.ws_bytes = pl.xa_bytes + (int64_t)pl.nrg * t->hidden * 16 * 4;
  return LRQ_OK;
}

}  // namespace lrq

extern "C" int64_t lrq_lora_grads_workspace(const lrq_tensors* t, int32_t n_out) {
  int st = lrq::validate_tensors(t);
  if (st) return st;
  lrq::LoraPlan pl;
  st = lrq::lora_plan(t, n_out, pl);
  return st ? st : pl.ws_bytes;
}

extern "C" int lrq_lora_grads(const lrq_tensors* t, const void* a, int64_t lda, const void* gmat, int64_t ldg,
                              int32_t n_out, void* xa, int64_t ldxa, int32_t xa_f32, void* da, int64_t ldda,
                              int32_t da_f32, void* workspace, int64_t workspace_bytes, void* stream) {
  using namespace lrq;
  int st = validate_tensors(t);
  if (st) return st;
  LoraPlan pl;
  st = lora_plan(t, n_out, pl);
  if (st) return st;
  if (a == nullptr || gmat == nullptr || xa == nullptr || da == nullptr) return LRQ_ERR_NULL;
  if (lda < n_out || ldg < n_out || ldxa < n_out || ldda < n_out) return LRQ_ERR_SHAPE;
  if (!aligned(a, 2) || ldg % 4 != 0 || !aligned(gmat, 8) || ldg * 2 >= (int64_t(1) << 24)) return LRQ_ERR_ALIGN;
  if (ldxa % 4 != 0 || !aligned(xa, xa_f32 ? 16 : 8) || ldda % 4 != 0 || !aligned(da, da_f32 ? 16 : 8))
    return LRQ_ERR_ALIGN;
  hipStream_t s = (hipStream_t)stream;
  if (t->rows == 0)  // da of no rows: zeros (no partials, no workspace)
    return launch(k_lora_sum, dim3((unsigned)((t->hidden * 4 + 255) / 256)), dim3(256), 0, s, (const float*)nullptr,
                  0, 0, xa, ldxa, xa_f32, (const float*)nullptr, 0, (int)t->hidden, da, ldda, da_f32);
  if (workspace == nullptr) return LRQ_ERR_NULL;
  if (workspace_bytes < pl.ws_bytes) return LRQ_ERR_WORKSPACE;
  if (!aligned(workspace, 16)) return LRQ_ERR_ALIGN;
  float* xa_part = reinterpret_cast<float*>(workspace);
  float* da_part = reinterpret_cast<float*>(reinterpret_cast<unsigned char*>(workspace) + pl.xa_bytes);
  auto go = [&](auto kern) {
    return launch(kern, dim3((unsigned)(pl.ncg * pl.nrg)), dim3(LoraGeo::NW * 64), 0, s, (const uint8_t*)t->codes,
                  t->ld_codes, (const uint16_t*)t->qparams, t->ld_qp, (const uint16_t*)t->L, t->ld_L,
                  (const uint16_t*)t->V, (int)t->rows, (int)t->hidden, (const uint16_t*)a, lda,
                  (const uint16_t*)gmat, ldg, xa_part, da_part, pl.bpg, pl.ncg);
  };
  switch (pl.nbw) {
    case 1: st = go(k_lora_grads<1>); break;
    case 2: st = go(k_lora_grads<2>); break;
    case 4: st = go(k_lora_grads<4>); break;
    case 8: st = go(k_lora_grads<8>); break;
    default: st = go(k_lora_grads<16>); break;
  }
  if (st) return st;
  const int64_t nq = ((int64_t)t->rows + t->hidden) * 4;
  return launch(k_lora_sum, dim3((unsigned)((nq + 255) / 256)), dim3(256), 0, s, (const float*)xa_part, pl.ncg,
                (int)t->rows, xa, ldxa, xa_f32, (const float*)da_part, pl.nrg, (int)t->hidden, da, ldda, da_f32);
}
