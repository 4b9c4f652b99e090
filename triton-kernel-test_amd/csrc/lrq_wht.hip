// Blockwise normalised Walsh-Hadamard rotation, 128 points (config 4's rotation, its own
// inverse): for every 128-column block b of a row,
//
//   y[128b + o] = bf16( fp32(S_o) * fp32(1/sqrt(128)) ),   S_o = sum_k H128[o, k] x[128b + k],
//
// with S_o accumulated on MFMA in four chained 32-term steps (each step adds 32 exact
// products to the running fp32 sum and rounds once).  Step c covers the columns
// 32g + 8c + e (g < 4, e < 8); the CPU oracle (wht128_rows) sums in the same order.
//
// Layout: a wave owns one 128-column block of 16 rows; lane (j, g) holds columns
// 32g .. 32g+31 of row j, which are both its B operands (step c = columns 32g + 8c ..) and,
// with output column o = 32g' + 4q + v assigned to MFMA tile q, lane (j, g') and element v,
// exactly where its outputs land, so no data moves between lanes.
//
// H128[o, k] = (-1)^popcount(o & k).  With o = (v, q, g') and k = (e, c, kg) in bit fields
// (2, 3, 2) and (3, 2, 2), the sign splits into a factor that depends on (v, g', e, kg, q0)
// (the lane's A operand for tile parity q0) and a wave-uniform factor (-1)^((q1&c0)^(q2&c1)):
// two register operands and their negations serve all 32 MFMAs of a block.
#include "lrq_common.h"
#include "lrq_host.h"
#include "lrq_whtop.h"

#include <algorithm>

namespace lrq {

// Grid: (ceil(row blocks / RBW), ceil(blocks per row / 4)); 4 waves, wave w on 128-column block
// blockIdx.y * 4 + w (idle past the end; no barrier follows).  In-place (x == y) is safe: a
// wave reads all of its rows' block before writing it.
template <int RBW>
__global__ __launch_bounds__(256) void k_wht128(const uint16_t* x, int64_t ldx, int M, int N, uint16_t* y,
                                                int64_t ldy) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int j = lane & 15, g = lane >> 4;
  const int blk = blockIdx.y * 4 + w;
  if (blk >= N / 128) return;
  const int nrb = (M + 15) / 16;
  u32x4 op[2][2];  // [q0][negated]
#pragma unroll
  for (int q0 = 0; q0 < 2; ++q0)
#pragma unroll
    for (int n = 0; n < 2; ++n) op[q0][n] = wht_base_operand(j, g, q0, n != 0);
  const float kScale = 0.08838834764831845f;  // fp32(1/sqrt(128))

#pragma unroll 1
  for (int b = 0; b < RBW; ++b) {
    const int rb = blockIdx.x * RBW + b;
    if (rb >= nrb) break;  // uniform
    const int64_t row = min(rb * 16 + j, M - 1);
    const uint16_t* xr = x + row * ldx + 128 * blk + 32 * g;
    u32x4 xv[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) xv[c] = ld16(xr + 8 * c);
    float out[32];
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      f32x4 acc = zero4();
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int flip = (((q >> 1) & c & 1) ^ ((q >> 2) & (c >> 1) & 1));
        acc = mfma_16x16x32(op[q & 1][flip], xv[c], acc);
      }
#pragma unroll
      for (int v = 0; v < 4; ++v) out[4 * q + v] = acc[v] * kScale;
    }
    uint16_t* yr = y + row * ldy + 128 * blk + 32 * g;
#pragma unroll
    for (int k = 0; k < 4; ++k) st16(yr + 8 * k, pack8(out + 8 * k));
  }
}

// Row-persistent form for hidden % 512 == 0: a workgroup of 4 waves owns a 512-column slab
// (wave w: 128-column block w of the slab) for a range of row blocks.  Each block's 16 x 1 KB
// slice moves straight from HBM into an LDS tile (two tiles, block b in tile b&1), each wave
// reads its block in the lane layout above, rotates it and writes the result over the same
// positions; after the next barrier the workgroup stores the tile as whole 1 KB row segments
// (non-temporal, full lines).  Per block: wait for block b's loads + barrier -> store block
// b-1 -> barrier (its tile reads returned) -> load block b+1 into that tile -> rotate block b.
// In place (x == y) is safe: a block is stored only after all of it has been read, and other
// blocks touch other rows.  Rows past the end repeat the last row (identical stores).
__global__ __launch_bounds__(256) void k_wht_rows(const uint16_t* x, int64_t ldx, int M, uint16_t* y, int64_t ldy,
                                                  int RBW) {
  constexpr int PITCH = 1024 + 16, TILE = 16 * PITCH;
  __shared__ __attribute__((aligned(16))) unsigned char sm[2 * TILE];
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int j = lane & 15, g = lane >> 4;
  const int nrb = (M + 15) / 16;
  const int rb0 = blockIdx.x * RBW;
  if (rb0 >= nrb) return;  // whole workgroup
  const int nblk = min(RBW, nrb - rb0);
  const int64_t c0 = (int64_t)blockIdx.y * 512;  // slab's first column
  u32x4 op[2][2];  // [q0][negated]
#pragma unroll
  for (int q0 = 0; q0 < 2; ++q0)
#pragma unroll
    for (int n = 0; n < 2; ++n) op[q0][n] = wht_base_operand(j, g, q0, n != 0);
  const unsigned char* xb = reinterpret_cast<const unsigned char*>(x + c0);
  unsigned char* yb = reinterpret_cast<unsigned char*>(y + c0);
  auto dma = [&](int rb, int tb) {  // wave w loads rows 4w .. 4w+3
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = 4 * w + i;
      const int64_t row = min(rb * 16 + r, M - 1);
      ld16_to_lds(xb + row * ldx * 2 + lane * 16, sm + tb * TILE + r * PITCH);
    }
  };
  auto store_tile = [&](int rb, int tb) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int k = tid + 256 * i, r = k >> 6, c16 = k & 63;
      const u32x4 v = *reinterpret_cast<const u32x4*>(sm + tb * TILE + r * PITCH + c16 * 16);
      const int64_t row = min(rb * 16 + r, M - 1);
      st16_stream(yb + row * ldy * 2 + c16 * 16, v);
    }
  };
  auto rotate = [&](int tb) { wht128_lds(sm + tb * TILE + j * PITCH + (128 * w + 32 * g) * 2, op); };
  dma(rb0, 0);
#pragma unroll 1
  for (int b = 0; b < nblk; ++b) {
    const int tb = b & 1;
    // block b's loads are this wave's last memory operations (vmcnt retires in issue order)
    __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0)
    lds_barrier();
    if (b > 0) store_tile(rb0 + b - 1, tb ^ 1);
    if (b + 1 < nblk) {
      lds_barrier();  // every wave's reads of tile tb^1 have returned
      __builtin_amdgcn_sched_barrier(0);
      dma(rb0 + b + 1, tb ^ 1);
      __builtin_amdgcn_sched_barrier(0);
    }
    rotate(tb);
  }
  lds_barrier();
  store_tile(rb0 + nblk - 1, (nblk - 1) & 1);
}

}  // namespace lrq

using namespace lrq;

extern "C" int lrq_wht128(const void* x, int64_t ldx, int64_t rows, int64_t hidden, void* y, int64_t ldy,
                          void* stream) {
  if (x == nullptr || y == nullptr) return LRQ_ERR_NULL;
  if (rows < 0 || hidden <= 0 || rows > INT32_MAX || hidden > INT32_MAX) return LRQ_ERR_SHAPE;
  if (hidden % 128 != 0 || ldx < hidden || ldy < hidden) return LRQ_ERR_SHAPE;
  if ((ldx % 8) != 0 || (ldy % 8) != 0 || !aligned(x, 16) || !aligned(y, 16)) return LRQ_ERR_ALIGN;
  if (x != y) {  // partial overlap would race
    const uintptr_t xa = (uintptr_t)x, ya = (uintptr_t)y;
    const uintptr_t xe = xa + (uintptr_t)((rows > 0 ? rows - 1 : 0) * ldx + hidden) * 2;
    const uintptr_t ye = ya + (uintptr_t)((rows > 0 ? rows - 1 : 0) * ldy + hidden) * 2;
    if (rows > 0 && xa < ye && ya < xe) return LRQ_ERR_SHAPE;
  } else if (ldx != ldy) {
    return LRQ_ERR_SHAPE;
  }
  if (rows == 0) return LRQ_OK;
  if (hidden % 512 == 0) {
    // about 4 workgroups per CU over (row ranges, 512-column slabs)
    const int nrb = (int)((rows + 15) / 16);
    const int slabs = (int)(hidden / 512);
    const int ranges = std::max(1, std::min(nrb, cu_count() * 4 / slabs));
    const int rbw = (nrb + ranges - 1) / ranges;
    LRQ_TRY(launch(k_wht_rows, dim3((nrb + rbw - 1) / rbw, slabs), dim3(256), 0, (hipStream_t)stream,
                       (const uint16_t*)x, ldx, (int)rows, (uint16_t*)y, ldy, rbw));
    return LRQ_OK;
  }
  constexpr int RBW = 4;
  const int nrb = (int)((rows + 15) / 16);
  const int nblk = (int)(hidden / 128);
  dim3 grid((nrb + RBW - 1) / RBW, (nblk + 3) / 4);
  LRQ_TRY(launch((k_wht128<RBW>), grid, dim3(256), 0, (hipStream_t)stream, (const uint16_t*)x, ldx, (int)rows,
                     (int)hidden, (uint16_t*)y, ldy));
  return LRQ_OK;
}
