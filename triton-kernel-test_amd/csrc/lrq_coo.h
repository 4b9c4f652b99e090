// Internal interface of the outlier compaction (csrc/lrq_coo.hip) for the legacy encode.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace lrq {

// The argument checks of lrq_coo_compact (no HIP call): 0 or a negative LRQ_ERR_*.
int coo_compact_check(const void* o, int64_t B, int64_t M, int64_t N, int64_t* indices, int64_t ld_idx,
                      void* values, int64_t cap, int64_t* nnz, int64_t* piece_ptr, void* workspace,
                      int64_t workspace_bytes);

// The staged record of one 64-column piece (a row's columns 64c .. 64c+63), 8 bytes, that the
// legacy encode writes into piece_ptr[piece] in place of the piece's first-entry offset: the
// piece's entry count n and its first kCooSlots entries in column order, an entry being
// (column within the piece) | (bf16 bits << 16):
//   dword 0 = entry 0 | n << 8,   dword 1 = entry 1   (an absent entry is 0).
// A piece with n > kCooSlots also has its 64 dense values in the outlier tensor, from which the
// compaction takes its entries; the dense values of the other pieces are not written.
constexpr int kCooSlots = 2;
__host__ __device__ constexpr uint32_t coo_record_count(uint32_t dword0) { return (dword0 >> 8) & 0xffu; }

// The compaction of staged records: piece_ptr[0 .. B*M*ceil(N/64)) holds every piece's record
// (N % 64 == 0); the chunk totals, the chunk scan and the scatter follow, the scatter replacing
// each record by the piece's first-entry offset.  Arguments as checked by coo_compact_check.
int coo_compact_staged(const void* o, int64_t B, int64_t M, int64_t N, int64_t* indices, int64_t ld_idx,
                       void* values, int64_t cap, int64_t* nnz, int64_t* piece_ptr, void* workspace,
                       hipStream_t stream);

}  // namespace lrq
