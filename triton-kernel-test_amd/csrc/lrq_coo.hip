// Dense -> COO compaction of the legacy format's outliers.
//
// The reference returns the encode's outliers as `o.to_sparse()`
// (low_rank_extraction_fuse_compression_quantization.py:149): a coalesced COO tensor whose
// entry count the host must learn before it can allocate, a device -> host synchronisation in
// the middle of the encode.  Here the compaction runs on the GPU in three stream-ordered
// kernels and the count stays on the device:
//
//   k_coo_count   a workgroup per chunk of kChunk pieces (a piece = 64 columns of one row,
//                 8 lanes x 8 columns): nonzeros per piece into LDS, an exclusive scan over
//                 the chunk, the piece offsets within the chunk into piece_ptr and the chunk
//                 total into the workspace.
//   k_coo_scan    one workgroup: exclusive scan of the chunk totals (64-bit), nnz.
//   k_coo_scatter the count kernel's mapping again: each lane's nonzeros go to
//                 chunk offset + piece offset + its rank among the piece's 8 lanes, in column
//                 order, so the entries come out in row-major order (coalesced); piece_ptr
//                 becomes global.  Entries at positions >= cap are not written.
//
// piece_ptr[row * npc + c / 64] is the first entry of the piece holding column c of a row
// (npc = ceil(N / 64) pieces per row; piece_ptr[rows * npc] = nnz): the legacy decode reads
// the outliers of a 64-column piece from it without a dense tensor.  A value is an entry when
// its bf16 bits are not +0 or -0 (what to_sparse keeps of a bf16 tensor).
//
// After the legacy encode, which stages each piece's count and first entries as a record in
// piece_ptr (lrq_coo.h), the compaction is k_coo_totals (the chunk totals from the records) and
// k_coo_scatter_staged (the chunk scan, or k_coo_scan before it above kScanInline chunks; the
// entries from the records, and from the dense values only for pieces with more entries than a
// record holds).
#include "lrq_common.h"
#include "lrq_coo.h"
#include "lrq_host.h"

namespace lrq {

constexpr int kPiece = 64;
constexpr int kChunk = 4096;  // pieces per chunk
constexpr int kCooThreads = 1024;
constexpr int kStage = 8 * kPiece;  // entries a wave gathers in LDS (k_coo_scatter: its 8 pieces' worst case)
constexpr int kScanInline = 4096;   // chunks up to which the staged scatter sums the chunk totals itself
constexpr int kScatterThreads = 512;  // the staged scatter's workgroup (half a chunk)

// Exclusive prefix sum over the NT threads of the workgroup; returns the total in `total`.
template <int NT = kCooThreads>
__device__ __forceinline__ uint32_t coo_block_scan(uint32_t v, uint32_t* wsum, uint32_t& total) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  uint32_t incl = v;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const uint32_t o = __shfl_up(incl, d);
    if (lane >= d) incl += o;
  }
  if (lane == 63) wsum[w] = incl;
  __syncthreads();
  uint32_t before = 0, all = 0;
#pragma unroll
  for (int i = 0; i < NT / 64; ++i) {
    const uint32_t t = wsum[i];
    before += i < w ? t : 0u;
    all += t;
  }
  __syncthreads();
  total = all;
  return before + incl - v;
}

// The nonzero mask of the 8 columns col0 .. col0+7 of one row (bit i: column col0 + i), and
// their bf16 bits.  VEC: the row is 16-byte aligned and N % 8 == 0, so one 16-byte load.  The
// loads are unconditional (clamped addresses, values past the row dropped afterwards): a load
// under a per-lane branch would make the compiler wait for every load in flight at the join.
template <bool VEC>
__device__ __forceinline__ uint32_t coo_lane_mask(const uint16_t* __restrict__ row, int64_t col0, int64_t N,
                                                  uint32_t (&v)[4]) {
  if (VEC) {
    const bool in = col0 < N;
    const u32x4 w = ld16(row + (in ? col0 : N - 8));
    v[0] = in ? w[0] : 0u, v[1] = in ? w[1] : 0u, v[2] = in ? w[2] : 0u, v[3] = in ? w[3] : 0u;
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t c = col0 + 2 * i;
      const uint32_t lo = row[min(c, N - 1)], hi = row[min(c + 1, N - 1)];
      v[i] = (c < N ? lo : 0u) | (c + 1 < N ? hi << 16 : 0u);
    }
  }
  uint32_t m = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    m |= ((v[i] & 0x7fffu) != 0u ? 1u : 0u) << (2 * i);
    m |= ((v[i] & 0x7fff0000u) != 0u ? 1u : 0u) << (2 * i + 1);
  }
  return m;
}

// Row offset and piece-in-row of chunk-local piece `local`: 32-bit arithmetic (rem0 < npc <=
// 2^25, local < kChunk), the chunk's first row and remainder computed once.
__device__ __forceinline__ void piece_rc(uint32_t rem0, uint32_t npc, uint32_t local, uint32_t& dr, uint32_t& pcol) {
  const uint32_t t1 = rem0 + local;
  dr = t1 / npc;
  pcol = t1 - dr * npc;
}

template <bool VEC>
__global__ __launch_bounds__(kCooThreads) void k_coo_count(const uint16_t* __restrict__ o, int64_t N, int64_t npc,
                                                           int64_t npieces, int64_t* __restrict__ piece_ptr,
                                                           uint32_t* __restrict__ chunk_total) {
  __shared__ uint32_t cnt[kChunk];
  __shared__ uint32_t wsum[kCooThreads / 64];
  const int t = threadIdx.x, q = t & 7;
  const int64_t pc0 = (int64_t)blockIdx.x * kChunk;
  const int64_t row0 = pc0 / npc;
  const uint32_t rem0 = (uint32_t)(pc0 - row0 * npc), npc32 = (uint32_t)npc;
  // UN iterations' loads are issued before any of them is counted
  constexpr int UN = 8, IT = kChunk / (kCooThreads / 8);
  static_assert(IT % UN == 0, "unroll");
  for (int it0 = 0; it0 < IT; it0 += UN) {
    uint32_t m[UN];
#pragma unroll
    for (int u = 0; u < UN; ++u) {
      const uint32_t local = (it0 + u) * (kCooThreads / 8) + (t >> 3);
      const uint32_t lc = (uint32_t)min((int64_t)local, npieces - 1 - pc0);  // clamped: loaded, not counted
      uint32_t dr, pcol;
      piece_rc(rem0, npc32, lc, dr, pcol);
      uint32_t v[4];
      m[u] = coo_lane_mask<VEC>(o + (row0 + dr) * N, (int64_t)pcol * kPiece + 8 * q, N, v);
      m[u] = pc0 + local < npieces ? m[u] : 0u;
    }
#pragma unroll
    for (int u = 0; u < UN; ++u) {
      uint32_t n = __builtin_popcount(m[u]);
      n += __shfl_xor(n, 1);
      n += __shfl_xor(n, 2);
      n += __shfl_xor(n, 4);
      if (q == 0) cnt[(it0 + u) * (kCooThreads / 8) + (t >> 3)] = n;
    }
  }
  __syncthreads();
  constexpr int PPT = kChunk / kCooThreads;  // pieces per thread in the scan
  uint32_t c[PPT], s = 0;
#pragma unroll
  for (int i = 0; i < PPT; ++i) {
    c[i] = cnt[t * PPT + i];
    s += c[i];
  }
  uint32_t total;
  uint32_t off = coo_block_scan(s, wsum, total);
#pragma unroll
  for (int i = 0; i < PPT; ++i) {
    const int64_t pc = pc0 + t * PPT + i;
    if (pc < npieces) piece_ptr[pc] = off;
    off += c[i];
  }
  if (t == 0) chunk_total[blockIdx.x] = total;
}

// The chunk totals of staged records (the legacy encode's, lrq_coo.h): per chunk, the sum of its
// pieces' counts, and of its first kChunk / 2 pieces' (half_total), into the workspace; 8 bytes
// read per piece.  A workgroup of kTotalsThreads per chunk, thread t summing pieces
// t + kTotalsThreads i, i < 16 (16 coalesced loads in flight), so that several chunks'
// workgroups share a CU.
constexpr int kTotalsThreads = 256;
__global__ __launch_bounds__(kTotalsThreads) void k_coo_totals(const int64_t* __restrict__ piece_ptr, int64_t npieces,
                                                               uint32_t* __restrict__ chunk_total,
                                                               uint32_t* __restrict__ half_total) {
  constexpr int PPT = kChunk / kTotalsThreads, NW = kTotalsThreads / 64;
  static_assert(PPT % 2 == 0, "whole iterations per half");
  __shared__ uint32_t wsum[2][NW];
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  const int64_t pc0 = (int64_t)blockIdx.x * kChunk + t;
  uint32_t d0[PPT];
#pragma unroll
  for (int i = 0; i < PPT; ++i)  // clamped: loaded, not counted
    d0[i] = (uint32_t)piece_ptr[min(pc0 + (int64_t)kTotalsThreads * i, npieces - 1)];
  // the first half is iterations 0 .. PPT / 2 - 1
  uint32_t s = 0, f = 0;
#pragma unroll
  for (int i = 0; i < PPT; ++i) {
    const uint32_t c = pc0 + (int64_t)kTotalsThreads * i < npieces ? coo_record_count(d0[i]) : 0u;
    s += c;
    f += i < PPT / 2 ? c : 0u;
  }
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    s += __shfl_xor(s, d);
    f += __shfl_xor(f, d);
  }
  if (lane == 0) {
    wsum[0][w] = s;
    wsum[1][w] = f;
  }
  __syncthreads();
  if (t == 0) {
    uint32_t total = 0, first = 0;
#pragma unroll
    for (int i = 0; i < NW; ++i) {
      total += wsum[0][i];
      first += wsum[1][i];
    }
    chunk_total[blockIdx.x] = total;
    half_total[blockIdx.x] = first;
  }
}

// One workgroup: chunk_off[c] = sum of the totals of chunks < c; nnz and piece_ptr[npieces].
__global__ __launch_bounds__(kCooThreads) void k_coo_scan(const uint32_t* __restrict__ chunk_total, int64_t nchunks,
                                                          uint64_t* __restrict__ chunk_off, int64_t npieces,
                                                          int64_t* __restrict__ piece_ptr, int64_t* __restrict__ nnz) {
  __shared__ uint32_t wsum[kCooThreads / 64];
  uint64_t base = 0;
  for (int64_t c0 = 0; c0 < nchunks; c0 += kCooThreads) {
    const int64_t c = c0 + threadIdx.x;
    const uint32_t v = c < nchunks ? chunk_total[c] : 0u;
    uint32_t total;
    const uint32_t off = coo_block_scan(v, wsum, total);  // < 2^32: 1024 chunks of <= 2^18 entries
    if (c < nchunks) chunk_off[c] = base + off;
    base += total;
  }
  if (threadIdx.x == 0) {
    piece_ptr[npieces] = (int64_t)base;
    nnz[0] = (int64_t)base;
  }
}

// Branch-free predicated stores into a wave-uniform region of `len` bytes (an offset past it is
// dropped by the hardware): the entries are written without per-lane branches, so the loads of
// the next pieces stay in flight.
__device__ __forceinline__ void st8_region(void* base, uint32_t len, uint32_t off, uint64_t v, bool keep) {
  const __amdgpu_buffer_rsrc_t r = uniform_rsrc(base, len);
  __builtin_amdgcn_raw_buffer_store_b64(u32x2{(uint32_t)v, (uint32_t)(v >> 32)}, r, keep ? off : 0x7ffffff0u, 0, 0);
}
__device__ __forceinline__ void st2_region(void* base, uint32_t len, uint32_t off, uint16_t v, bool keep) {
  const __amdgpu_buffer_rsrc_t r = uniform_rsrc(base, len);
  __builtin_amdgcn_raw_buffer_store_b16(v, r, keep ? off : 0x7ffffff0u, 0, 0);
}

// The same stores through a buffer resource made once (uniform_rsrc) for several of them.
__device__ __forceinline__ void st8_at(__amdgpu_buffer_rsrc_t r, uint32_t off, uint64_t v, bool keep) {
  __builtin_amdgcn_raw_buffer_store_b64(u32x2{(uint32_t)v, (uint32_t)(v >> 32)}, r, keep ? off : 0x7ffffff0u, 0, 0);
}
__device__ __forceinline__ void st2_at(__amdgpu_buffer_rsrc_t r, uint32_t off, uint16_t v, bool keep) {
  __builtin_amdgcn_raw_buffer_store_b16(v, r, keep ? off : 0x7ffffff0u, 0, 0);
}

template <bool VEC>
__global__ __launch_bounds__(kCooThreads) void k_coo_scatter(const uint16_t* __restrict__ o, int64_t M, int64_t N,
                                                             int64_t npc, int64_t npieces,
                                                             int64_t* __restrict__ piece_ptr,
                                                             const uint64_t* __restrict__ chunk_off,
                                                             const uint32_t* __restrict__ chunk_total,
                                                             int64_t* __restrict__ idx, int64_t ld_idx,
                                                             uint16_t* __restrict__ val, int64_t cap) {
  // per wave: up to 8 pieces x 64 entries; entry = (row offset, column, value bits)
  __shared__ u32x4 stage[kCooThreads / 64][kStage];
  const int t = threadIdx.x, q = t & 7, lane = t & 63, w = t >> 6;
  const int64_t pc0 = (int64_t)blockIdx.x * kChunk;
  const int64_t coff = (int64_t)chunk_off[blockIdx.x];
  const int64_t row0 = pc0 / npc;
  const uint32_t rem0 = (uint32_t)(pc0 - row0 * npc), npc32 = (uint32_t)npc;
  const int64_t b0 = row0 / M;
  const uint32_t m0 = (uint32_t)(row0 - b0 * M), M32 = (uint32_t)M;
  // the chunk's entries are positions coff .. coff + total - 1; the part below cap is written
  const int64_t nw = max((int64_t)0, min((int64_t)chunk_total[blockIdx.x], cap - coff));
  const uint32_t len8 = (uint32_t)(nw * 8), len2 = (uint32_t)(nw * 2);
  int64_t* ib = idx + min(coff, cap);
  int64_t* im = ib + ld_idx;
  int64_t* in = im + ld_idx;
  uint16_t* vb = val + min(coff, cap);
  const uint32_t plen8 = (uint32_t)(min((int64_t)kChunk, npieces - pc0) * 8);
  constexpr int UN = 4, IT = kChunk / (kCooThreads / 8);
  static_assert(IT % UN == 0, "unroll");
  for (int it0 = 0; it0 < IT; it0 += UN) {
    // loads of UN pieces first (masks, values, piece offsets), then their entries
    uint32_t mu[UN], vu[UN][4], dru[UN], pcu[UN];
    int64_t lo[UN];
#pragma unroll
    for (int u = 0; u < UN; ++u) {
      const uint32_t local = (uint32_t)min((int64_t)(it0 + u) * (kCooThreads / 8) + (t >> 3), npieces - 1 - pc0);
      piece_rc(rem0, npc32, local, dru[u], pcu[u]);
      mu[u] = coo_lane_mask<VEC>(o + (row0 + dru[u]) * N, (int64_t)pcu[u] * kPiece + 8 * q, N, vu[u]);
      lo[u] = piece_ptr[pc0 + local];
    }
#pragma unroll
    for (int u = 0; u < UN; ++u) {
      const int64_t pc = pc0 + (it0 + u) * (kCooThreads / 8) + (t >> 3);
      const bool live = pc < npieces;  // past the last piece: a clamped duplicate, written nowhere
      const uint32_t m = live ? mu[u] : 0u;
      // rank of this lane's first entry among the piece's 8 lanes (lanes 8k .. 8k+7 of the wave)
      const uint32_t n = __builtin_popcount(m);
      uint32_t incl = n;
#pragma unroll
      for (int d = 1; d < 8; d <<= 1) {
        const uint32_t up = __shfl_up(incl, d, 8);
        if (q >= d) incl += up;
      }
      // the wave's 8 pieces are consecutive, so its entries are positions wbase .. wbase + wcnt - 1;
      // wcnt is the sum of the lanes' counts (lanes past the last piece count nothing; their
      // clamped offsets must not be used for it)
      const uint32_t lo32 = (uint32_t)lo[u];
      const uint32_t wbase = __shfl(lo32, 0);
      uint32_t wcnt = n;
#pragma unroll
      for (int d = 1; d < 64; d <<= 1) wcnt += __shfl_xor(wcnt, d);
      // stage the lane's entries (usually none) in the wave's LDS area at their rank, one set
      // bit at a time: only LDS stores sit under this per-lane loop, so no memory load waits
      uint32_t rel = lo32 + (incl - n) - wbase;
      uint32_t mm = m;
      while (mm != 0u) {
        const int i = __builtin_ctz(mm);
        mm &= mm - 1u;
        const uint32_t word = i < 2 ? vu[u][0] : i < 4 ? vu[u][1] : i < 6 ? vu[u][2] : vu[u][3];
        stage[w][rel++] = u32x4{dru[u], pcu[u] * kPiece + 8 * q + i, (word >> (16 * (i & 1))) & 0xffffu, 0u};
      }
      __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): the wave's LDS writes are done
      __builtin_amdgcn_wave_barrier();
      // write them out coalesced: lane e of each round takes entry e
      const uint32_t nround = __builtin_amdgcn_readfirstlane((wcnt + 63) / 64);
      for (uint32_t r = 0; r < nround; ++r) {
        const uint32_t e = r * 64 + lane;
        const u32x4 en = stage[w][min(e, (uint32_t)kStage - 1)];
        const uint32_t mr = m0 + en[0], qb = mr / M32;
        const bool keep = e < wcnt;
        const uint32_t off = wbase + e;
        st8_region(ib, len8, off * 8, (uint64_t)(b0 + qb), keep);
        st8_region(im, len8, off * 8, (uint64_t)(mr - qb * M32), keep);
        st8_region(in, len8, off * 8, (uint64_t)en[1], keep);
        st2_region(vb, len2, off * 2, (uint16_t)en[2], keep);
      }
      __builtin_amdgcn_wave_barrier();  // the area is reused by the next piece
      // the piece's global first entry (the store's value depends on the lanes' reads of it)
      st8_region(piece_ptr + pc0, plen8, (uint32_t)(pc - pc0) * 8, (uint64_t)(coff + lo[u]), q == 0 && live);
    }
  }
}

// The scatter of staged records (lrq_coo.h; N % 64 == 0), two workgroups of kScatterThreads per
// chunk, each over one half (a part: kChunk / 2 pieces), so that up to three of them share a CU.
// Up to kScanInline chunks it also does the chunk scan: each workgroup sums the totals of the
// chunks before its own (at most 16 KB from L2), and the first part of the last chunk writes nnz
// and piece_ptr[npieces]; above that k_coo_scan has run and chunk_off holds the chunk offsets.  The
// second part starts after the first's half_total entries.  Thread t of a part's workgroup owns its
// pieces 4t .. 4t+3, whose records it reads, scans over the workgroup (part-local first entries)
// and replaces by the global first entries.  A piece's entries go to its first entry + their rank:
// those a record holds, formed by the piece's thread; those of a piece with more entries, from its
// 64 dense values, by the wave eight pieces at a time (four such rounds' loads issued together).
// The wave's pieces are consecutive, so its entries are consecutive positions: up to kStage of them
// are gathered in the wave's LDS area at their position and written out coalesced (64 per store),
// more are written where they are formed.
__global__ __launch_bounds__(kScatterThreads) void k_coo_scatter_staged(
    const uint16_t* __restrict__ o, int64_t M, int64_t N, int64_t npc, int64_t npieces, int64_t nchunks,
    int64_t* __restrict__ piece_ptr, const uint64_t* __restrict__ chunk_off, const uint32_t* __restrict__ chunk_total,
    const uint32_t* __restrict__ half_total, int64_t* __restrict__ idx, int64_t ld_idx, uint16_t* __restrict__ val,
    int64_t cap, int64_t* __restrict__ nnz) {
  constexpr int NW = kScatterThreads / 64, PART = kChunk / 2, PPT = PART / kScatterThreads;
  __shared__ uint32_t wsum[NW];
  __shared__ uint64_t csum[NW];
  __shared__ u32x2 more_desc[NW][64 * PPT];  // per wave: (first entry, piece) of each such piece
  __shared__ u32x2 stage[NW][kStage];         // per wave: (column, row offset | bf16 bits << 16)
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  const int64_t chunk = blockIdx.x >> 1;
  const int part = blockIdx.x & 1;
  const int64_t pc0 = chunk * kChunk + part * PART;
  const int64_t np = min((int64_t)PART, npieces - pc0);  // pieces of the part
  if (np <= 0) return;  // the second part of a short last chunk (workgroup-uniform)
  // the records first (their loads overlap the chunk-offset sum)
  uint32_t d0[PPT], d1[PPT];
#pragma unroll
  for (int i = 0; i < PPT; ++i) {
    const uint32_t local = (uint32_t)min((int64_t)(PPT * t + i), np - 1);  // clamped: loaded, not counted
    const uint64_t rec = (uint64_t)piece_ptr[pc0 + local];
    d0[i] = (uint32_t)rec;
    d1[i] = (uint32_t)(rec >> 32);
  }
  // coff = the totals of chunks 0 .. chunk - 1 (+ the first part's, for the second)
  const bool inline_scan = chunk_off == nullptr;
  uint64_t part_sum = 0;
  if (inline_scan)
    for (int64_t c = t; c < chunk; c += kScatterThreads) part_sum += chunk_total[c];
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) part_sum += __shfl_xor(part_sum, d);
  if (lane == 0) csum[w] = part_sum;
  uint32_t c[PPT], s = 0;
#pragma unroll
  for (int i = 0; i < PPT; ++i) {
    c[i] = PPT * t + i < np ? coo_record_count(d0[i]) : 0u;
    s += c[i];
  }
  uint32_t total;
  uint32_t loc[PPT];
  loc[0] = coo_block_scan<kScatterThreads>(s, wsum, total);  // (its barriers also publish csum)
  int64_t chunk_start = 0;
#pragma unroll
  for (int i = 0; i < NW; ++i) chunk_start += (int64_t)csum[i];
  if (!inline_scan) chunk_start = (int64_t)chunk_off[chunk];
  const int64_t coff = chunk_start + (part ? (int64_t)half_total[chunk] : 0);
#pragma unroll
  for (int i = 1; i < PPT; ++i) loc[i] = loc[i - 1] + c[i - 1];
  if (inline_scan && chunk == nchunks - 1 && part == 0 && t == 0) {
    const uint64_t all = (uint64_t)(chunk_start + chunk_total[chunk]);
    st8_region(piece_ptr + npieces, 8, 0, all, true);
    st8_region(nnz, 8, 0, all, true);
  }
  const int64_t row0 = pc0 / npc;
  const uint32_t rem0 = (uint32_t)(pc0 - row0 * npc), npc32 = (uint32_t)npc;
  const int64_t b0 = row0 / M;
  const uint32_t m0 = (uint32_t)(row0 - b0 * M), M32 = (uint32_t)M;
  // the chunk's entries are positions coff .. coff + total - 1; the part below cap is written
  const int64_t nw = max((int64_t)0, min((int64_t)total, cap - coff));
  const uint32_t len8 = (uint32_t)(nw * 8), len2 = (uint32_t)(nw * 2);
  int64_t* ib = idx + min(coff, cap);
  int64_t* im = ib + ld_idx;
  int64_t* in = im + ld_idx;
  uint16_t* vb = val + min(coff, cap);
  const uint32_t plen8 = (uint32_t)(np * 8);
  // the regions' buffer resources, made once
  const __amdgpu_buffer_rsrc_t r_ib = uniform_rsrc(ib, len8), r_im = uniform_rsrc(im, len8),
                               r_in = uniform_rsrc(in, len8), r_vb = uniform_rsrc(vb, len2),
                               r_pp = uniform_rsrc(piece_ptr + pc0, plen8);
  // each thread rewrites only the records it read
#pragma unroll
  for (int i = 0; i < PPT; ++i) st8_at(r_pp, (uint32_t)(PPT * t + i) * 8, (uint64_t)(coff + loc[i]), true);
  // the row (from row0) and 64-column piece of each of the thread's pieces: one division, then steps
  uint32_t dr[PPT], pcol[PPT];
  piece_rc(rem0, npc32, (uint32_t)min((int64_t)(PPT * t), np - 1), dr[0], pcol[0]);
#pragma unroll
  for (int i = 1; i < PPT; ++i) {
    dr[i] = dr[i - 1];
    pcol[i] = pcol[i - 1] + 1u;
    if (pcol[i] == npc32) {
      pcol[i] = 0u;
      ++dr[i];
    }
  }
  // batch and row of a row offset: one batch for the whole part unless it crosses a batch end
  uint32_t dr_last, pc_last;
  piece_rc(rem0, npc32, (uint32_t)(np - 1), dr_last, pc_last);
  const bool one_batch = m0 + dr_last < M32;
  auto batch_row = [&](uint32_t d, uint64_t& b, uint64_t& m) __attribute__((always_inline)) {
    const uint32_t mr = m0 + d, qb = one_batch ? 0u : mr / M32;
    b = (uint64_t)(b0 + qb);
    m = (uint64_t)(mr - qb * M32);
  };
  // the wave's pieces are consecutive: its entries are part positions wbase .. wbase + wtot - 1
  const uint32_t wbase = __builtin_amdgcn_readlane(loc[0], 0);
  const uint32_t wtot = __builtin_amdgcn_readlane(loc[PPT - 1] + c[PPT - 1], 63) - wbase;
  // the pieces with more entries than a record holds, listed per wave (first entry, piece)
  uint32_t nmore = 0;
#pragma unroll
  for (int i = 0; i < PPT; ++i) {
    const bool more = c[i] > (uint32_t)kCooSlots;
    const uint64_t bal = __builtin_amdgcn_ballot_w64(more);
    const uint32_t r = nmore + __builtin_amdgcn_mbcnt_hi((uint32_t)(bal >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)bal, 0u));
    if (more) more_desc[w][r] = u32x2{loc[i], (uint32_t)(PPT * t + i)};
    nmore += (uint32_t)__builtin_popcountll(bal);
  }
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): the wave's LDS writes are done
  __builtin_amdgcn_wave_barrier();
  // Every entry goes through sink(part position, row offset, column, bf16 bits, keep): the entries a
  // record holds from the piece's thread; those of the listed pieces from their dense values, eight
  // pieces at a time (lane 8p + q: columns 8q .. 8q+7 of the round's piece p, ranks by a scan over
  // the piece's 8 lanes).
  auto entries = [&](auto sink) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < PPT; ++i)
#pragma unroll
      for (int k = 0; k < kCooSlots; ++k) {
        const bool keep = c[i] <= (uint32_t)kCooSlots && (uint32_t)k < c[i];
        if (__builtin_amdgcn_ballot_w64(keep) == 0) continue;  // wave-uniform
        const uint32_t dw = k == 0 ? d0[i] : d1[i];
        sink(loc[i] + k, dr[i], pcol[i] * kPiece + (dw & 63u), dw >> 16, keep);
      }
    const int q = lane & 7;
    constexpr int RA = 4;  // rounds whose loads are in flight together
    for (uint32_t r0 = 0; r0 < nmore; r0 += 8 * RA) {
      u32x4 v[RA];
      uint32_t pdr[RA], ppc[RA], first[RA];
#pragma unroll
      for (int j = 0; j < RA; ++j) {  // (rounds past the list load a listed piece again: unused)
        const u32x2 desc = more_desc[w][min(r0 + 8 * j + (uint32_t)(lane >> 3), nmore - 1)];
        first[j] = desc[0];
        piece_rc(rem0, npc32, desc[1], pdr[j], ppc[j]);
        v[j] = ld16(o + (row0 + pdr[j]) * N + (int64_t)ppc[j] * kPiece + 8 * q);
      }
#pragma unroll
      for (int j = 0; j < RA; ++j) {
        if (r0 + 8 * j >= nmore) break;  // wave-uniform
        const bool live = r0 + 8 * j + (uint32_t)(lane >> 3) < nmore;
        uint32_t m = 0;
#pragma unroll
        for (int h = 0; h < 4; ++h) {
          m |= ((v[j][h] & 0x7fffu) != 0u ? 1u : 0u) << (2 * h);
          m |= ((v[j][h] & 0x7fff0000u) != 0u ? 1u : 0u) << (2 * h + 1);
        }
        m = live ? m : 0u;
        const uint32_t n = __builtin_popcount(m);
        uint32_t incl = n;
#pragma unroll
        for (int d = 1; d < 8; d <<= 1) {
          const uint32_t up = __shfl_up(incl, d, 8);
          if (q >= d) incl += up;
        }
        uint32_t off = first[j] + incl - n;
        while (__builtin_amdgcn_ballot_w64(m != 0u) != 0) {
          const bool keep = m != 0u;
          const uint32_t i = __builtin_ctz(m | 0x100u) & 7u;
          m &= m - 1u;
          const u32x4 vj = v[j];
          const uint32_t word = (i & 4u) ? ((i & 2u) ? vj[3] : vj[2]) : ((i & 2u) ? vj[1] : vj[0]);
          sink(off, pdr[j], ppc[j] * kPiece + 8u * q + i, (word >> (16u * (i & 1u))) & 0xffffu, keep);
          off += keep ? 1u : 0u;
        }
      }
    }
  };
  if (wtot <= (uint32_t)kStage) {  // wave-uniform
    // the entries into the wave's LDS area at their position, then written out coalesced
    entries([&](uint32_t off, uint32_t d, uint32_t col, uint32_t bits, bool keep) __attribute__((always_inline)) {
      if (keep) stage[w][off - wbase] = u32x2{col, d | bits << 16};
    });
    __builtin_amdgcn_s_waitcnt(0xc07f);
    __builtin_amdgcn_wave_barrier();
    for (uint32_t r0 = 0; r0 < wtot; r0 += 64) {
      const uint32_t e = r0 + lane;
      const bool keep = e < wtot;
      const u32x2 en = stage[w][min(e, (uint32_t)kStage - 1)];
      uint64_t b, m;
      batch_row(en[1] & 0xffffu, b, m);
      const uint32_t off = wbase + e;
      st8_at(r_ib, off * 8, b, keep);
      st8_at(r_im, off * 8, m, keep);
      st8_at(r_in, off * 8, (uint64_t)en[0], keep);
      st2_at(r_vb, off * 2, (uint16_t)(en[1] >> 16), keep);
    }
  } else {
    // more entries than the area holds: each written where it is formed
    entries([&](uint32_t off, uint32_t d, uint32_t col, uint32_t bits, bool keep) __attribute__((always_inline)) {
      uint64_t b, m;
      batch_row(d, b, m);
      st8_at(r_ib, off * 8, b, keep);
      st8_at(r_im, off * 8, m, keep);
      st8_at(r_in, off * 8, (uint64_t)col, keep);
      st2_at(r_vb, off * 2, (uint16_t)bits, keep);
    });
  }
}

struct CooPlan {
  int64_t npc, npieces, nchunks, ws_bytes;
};

static CooPlan coo_plan(int64_t B, int64_t M, int64_t N) {
  CooPlan p{};
  p.npc = (N + kPiece - 1) / kPiece;
  p.npieces = B * M * p.npc;
  p.nchunks = (p.npieces + kChunk - 1) / kChunk;
  p.ws_bytes = p.nchunks * 16;  // uint64 offsets, uint32 totals, uint32 first-half totals (staged path)
  return p;
}

}  // namespace lrq

using namespace lrq;

extern "C" int64_t lrq_coo_workspace(int64_t B, int64_t M, int64_t N) {
  if (B < 0 || M < 0 || N <= 0) return LRQ_ERR_SHAPE;
  return coo_plan(B, M, N).ws_bytes;
}

int lrq::coo_compact_check(const void* o, int64_t B, int64_t M, int64_t N, int64_t* indices, int64_t ld_idx,
                           void* values, int64_t cap, int64_t* nnz, int64_t* piece_ptr, void* workspace,
                           int64_t workspace_bytes) {
  if (o == nullptr || nnz == nullptr || piece_ptr == nullptr) return LRQ_ERR_NULL;
  if (B < 0 || M < 0 || N <= 0 || cap < 0 || ld_idx < cap) return LRQ_ERR_SHAPE;
  if (M > INT32_MAX || N > INT32_MAX) return LRQ_ERR_SHAPE;  // 32-bit row / piece arithmetic
  if (cap > 0 && (indices == nullptr || values == nullptr)) return LRQ_ERR_NULL;
  if (!aligned(o, 2) || !aligned(indices, 8) || !aligned(values, 2) || !aligned(nnz, 8) || !aligned(piece_ptr, 8))
    return LRQ_ERR_ALIGN;
  const CooPlan p = coo_plan(B, M, N);
  if (p.nchunks > ((int64_t)1 << 31) - 1) return LRQ_ERR_SHAPE;
  if (p.nchunks > 0) {
    if (workspace == nullptr) return LRQ_ERR_NULL;
    if (workspace_bytes < p.ws_bytes) return LRQ_ERR_WORKSPACE;
    if (!aligned(workspace, 8)) return LRQ_ERR_ALIGN;
  }
  return LRQ_OK;
}

// The chunk scan and the scatter (after the count pass).
static int coo_scan_scatter(const uint16_t* ob, int64_t M, int64_t N, const CooPlan& p, int64_t* indices,
                            int64_t ld_idx, void* values, int64_t cap, int64_t* nnz, int64_t* piece_ptr,
                            uint64_t* chunk_off, uint32_t* chunk_total, bool vec, hipStream_t s) {
  LRQ_TRY(launch(k_coo_scan, dim3(1), dim3(kCooThreads), 0, s, chunk_total, p.nchunks, chunk_off, p.npieces,
                     piece_ptr, nnz));
  if (p.nchunks > 0) {
    if (vec) LRQ_TRY(launch(k_coo_scatter<true>, dim3((unsigned)p.nchunks), dim3(kCooThreads), 0, s, ob, M, N,
                                p.npc, p.npieces, piece_ptr, chunk_off, chunk_total, indices, ld_idx,
                                (uint16_t*)values, cap));
    else LRQ_TRY(launch(k_coo_scatter<false>, dim3((unsigned)p.nchunks), dim3(kCooThreads), 0, s, ob, M, N,
                            p.npc, p.npieces, piece_ptr, chunk_off, chunk_total, indices, ld_idx, (uint16_t*)values,
                            cap));
  }
  return LRQ_OK;
}

int lrq::coo_compact_staged(const void* o, int64_t B, int64_t M, int64_t N, int64_t* indices, int64_t ld_idx,
                            void* values, int64_t cap, int64_t* nnz, int64_t* piece_ptr, void* workspace,
                            hipStream_t s) {
  const CooPlan p = coo_plan(B, M, N);
  if (N % kPiece != 0 || p.nchunks == 0) return LRQ_ERR_SHAPE;  // whole pieces, at least one
  uint64_t* chunk_off = reinterpret_cast<uint64_t*>(workspace);
  uint32_t* chunk_total = reinterpret_cast<uint32_t*>(chunk_off + p.nchunks);
  uint32_t* half_total = chunk_total + p.nchunks;  // the workspace's last nchunks * 4 bytes
  LRQ_TRY(launch(k_coo_totals, dim3((unsigned)p.nchunks), dim3(kTotalsThreads), 0, s, piece_ptr, p.npieces,
                 chunk_total, half_total));
  const bool inline_scan = p.nchunks <= kScanInline;
  if (!inline_scan)
    LRQ_TRY(launch(k_coo_scan, dim3(1), dim3(kCooThreads), 0, s, chunk_total, p.nchunks, chunk_off, p.npieces,
                   piece_ptr, nnz));
  LRQ_TRY(launch(k_coo_scatter_staged, dim3((unsigned)(2 * p.nchunks)), dim3(kScatterThreads), 0, s,
                 (const uint16_t*)o, M, N, p.npc, p.npieces, p.nchunks, piece_ptr, inline_scan ? nullptr : chunk_off,
                 chunk_total, half_total, indices, ld_idx, (uint16_t*)values, cap, nnz));
  return LRQ_OK;
}

extern "C" int lrq_coo_compact(const void* o, int64_t B, int64_t M, int64_t N, int64_t* indices, int64_t ld_idx,
                               void* values, int64_t cap, int64_t* nnz, int64_t* piece_ptr, void* workspace,
                               int64_t workspace_bytes, void* stream) {
  const int st = coo_compact_check(o, B, M, N, indices, ld_idx, values, cap, nnz, piece_ptr, workspace,
                                   workspace_bytes);
  if (st) return st;
  const CooPlan p = coo_plan(B, M, N);
  hipStream_t s = (hipStream_t)stream;
  uint64_t* chunk_off = reinterpret_cast<uint64_t*>(workspace);
  uint32_t* chunk_total = reinterpret_cast<uint32_t*>(chunk_off + p.nchunks);
  const bool vec = N % 8 == 0 && aligned(o, 16);
  const uint16_t* ob = (const uint16_t*)o;
  if (p.nchunks > 0) {
    if (vec) LRQ_TRY(launch(k_coo_count<true>, dim3((unsigned)p.nchunks), dim3(kCooThreads), 0, s, ob, N, p.npc,
                                p.npieces, piece_ptr, chunk_total));
    else LRQ_TRY(launch(k_coo_count<false>, dim3((unsigned)p.nchunks), dim3(kCooThreads), 0, s, ob, N, p.npc,
                            p.npieces, piece_ptr, chunk_total));
  }
  return coo_scan_scatter(ob, M, N, p, indices, ld_idx, values, cap, nnz, piece_ptr, chunk_off, chunk_total, vec, s);
}
