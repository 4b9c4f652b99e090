// Internal interface of the outlier compaction (csrc/lrq_coo.hip) for the legacy encode.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace lrq {

// The argument checks of lrq_coo_compact (no HIP call): 0 or a negative LRQ_ERR_*.
int coo_compact_check(const void* o, int64_t B, int64_t M, int64_t N, int64_t* indices, int64_t ld_idx,
                      void* values, int64_t cap, int64_t* nnz, int64_t* piece_ptr, void* workspace,
                      int64_t workspace_bytes);

// The compaction after its count pass: piece_ptr[0 .. B*M*ceil(N/64)) already holds every piece's
// entry count (as the legacy encode writes them); offsets, the chunk scan and the scatter follow.
// Arguments as checked by coo_compact_check.
int coo_compact_counted(const void* o, int64_t B, int64_t M, int64_t N, int64_t* indices, int64_t ld_idx,
                        void* values, int64_t cap, int64_t* nnz, int64_t* piece_ptr, void* workspace,
                        hipStream_t stream);

}  // namespace lrq
