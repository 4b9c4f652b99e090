/*
 * lrq.h — C ABI of the MI355X (gfx950) compressed-activation library (liblrq.so).
 *
 * The reference (Ther-nullptr/Triton-Kernel-Test) exposes this path as Python functions
 * over torch CUDA tensors that launch Triton kernels.  Each entry point below replaces one
 * of those launches; the reference function it stands in for is cited beside it.  The
 * Python package `triton-kernel-test_amd` keeps the reference's function names and
 * calls these through ctypes.
 *
 * Conventions (every entry point):
 *   - Pointers are device pointers (HBM) unless stated; dimensions and leading
 *     dimensions are int64 element counts; matrices are row-major.
 *   - bf16 / fp16 tensors are passed as raw 16-bit storage.
 *   - `stream` is a hipStream_t (NULL = the legacy default stream).  Work is enqueued
 *     asynchronously; nothing synchronises the host.
 *   - No entry point allocates device memory.  Outputs and workspaces come from the
 *     caller.  No global mutable state is kept: calls are reentrant and thread-safe.
 *   - Return value: LRQ_OK (0) on success; a negative LRQ_ERR_* when an argument is
 *     invalid — always detected on the host BEFORE any HIP call, so these paths can be
 *     exercised without a GPU; a positive hipError_t if a launch fails.
 *
 * Compressed format ("group mode", the north-star format).  An activation X[rows, hidden]
 * (bf16) is stored as
 *     L       bf16  [rows, rank]          projection coefficients, L = bf16(Y V)
 *     codes   uint8 [rows, hidden*bits/8] residual codes, row-planar packing: byte j of a
 *                                         row holds column j + i*hidden*bits/8 in bits
 *                                         [bits*i, bits*i + bits), i < NP = 8/bits
 *     qparams fp16  [rows, U, NP, 2]      U = hidden/(group*NP) units per row; entry
 *                                         [r, u, i] is (scale, zero) of the group of columns
 *                                         i*hidden/NP + u*group .. + group - 1 (the groups
 *                                         whose codes share bytes u*group .. + group - 1)
 *     side    fp16  [rows, n_outlier]     outlier channels kept dense (optional)
 *     idx     int32 [n_outlier]           their column indices (optional), distinct; an entry
 *                                         outside [0, hidden) is skipped by every kernel and
 *                                         its side column is not written
 * where Y = X (or its blockwise 128-point Walsh-Hadamard rotation) and V[hidden, rank] is
 * an orthonormal basis supplied by the caller.
 */
#ifndef LRQ_H
#define LRQ_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LRQ_OK 0
#define LRQ_ERR_NULL (-1)        /* a required pointer is NULL                         */
#define LRQ_ERR_SHAPE (-2)       /* a dimension or leading dimension is invalid        */
#define LRQ_ERR_UNSUPPORTED (-3) /* bits / group / rank / flag combination not built    */
#define LRQ_ERR_ALIGN (-4)       /* pointer or leading dimension misaligned             */
#define LRQ_ERR_WORKSPACE (-5)   /* caller workspace too small                          */

/* The rotated format (config 4) stores encode(bf16(WHT(x))) and decodes to
 * WHT(bf16(decode)).  The flag marks a descriptor as rotated.  lrq_encode with the flag reads
 * the unrotated x and rotates it as it reads (int4/g64 and int8/g128, no outlier channels,
 * hidden/NP a multiple of 128, an even number of units per row); for other shapes it returns
 * LRQ_ERR_UNSUPPORTED and the caller rotates x with lrq_wht128 into a buffer, then encodes
 * that with the flag cleared.  lrq_decode, the fused consumers and the dequant-GEMMs undo the
 * rotation (the dequant-GEMMs need planes of whole rotation blocks, hidden/NP a multiple of 128,
 * else LRQ_ERR_UNSUPPORTED); lrq_lora_grads refuses the flag (LRQ_ERR_UNSUPPORTED: use
 * lrq_dequant_gemm and lrq_dequant_gemm_t). */
#define LRQ_FLAG_HADAMARD 1

/* Descriptor of one compressed activation.  Encode writes L/codes/scale/zero/side;
 * decode-side entry points read them.  Unused fields may be NULL / 0. */
typedef struct lrq_tensors {
  int64_t rows, hidden;
  int32_t rank;  /* 0, 16 or 32 */
  int32_t bits;  /* 4 or 8 */
  int32_t group; /* 64 or 128 (multiple of 32) */
  int32_t flags; /* LRQ_FLAG_* */
  void* L;
  int64_t ld_L;
  const void* V;  /* bf16 [hidden, rank] */
  const void* Vt; /* bf16 [rank, hidden]; read only by the two-pass encode (rank 32 and hidden
                     sizes without a single-pass kernel); lrq_transpose_bf16 builds it */
  void* codes;
  int64_t ld_codes;
  void* qparams;  /* fp16 [rows, U, NP, 2], see above */
  int64_t ld_qp;  /* row stride of qparams in fp16 elements (>= 2*hidden/group) */
  const int32_t* outlier_idx;
  int32_t n_outlier;
  void* side;
  int64_t ld_side;
} lrq_tensors;

/* ------------------------------------------------------------------ group mode */

/* Encode X[rows, hidden] (bf16, leading dim ldx) into `t`.
 * Replaces low_rank_addition_fuse_compression_quantization
 * (low_rank_extraction_fuse_compression_quantization.py:118-150, kernel :13-115) in the
 * north-star format: projection, residual, per-group quantisation and packing in one pass
 * over X when hidden has a single-pass kernel, otherwise two passes. */
int lrq_encode(const lrq_tensors* t, const void* x, int64_t ldx, void* stream);

/* Decode `t` into out[rows, hidden] bf16.
 * Replaces low_rank_addition_fuse_decompression_dequantization
 * (low_rank_extraction_fuse_decompression_dequantization.py:116-152, kernel :13-113). */
int lrq_decode(const lrq_tensors* t, void* out, int64_t ldo, void* stream);

/* The four consumers below may write their output over their second input (dx == dy) except
 * where they run as a decode followed by a dense pass (the rotated format in shapes without a
 * fused rotated kernel; in lrq_softmax_bwd, outlier channels, and the rotated format with planes
 * that are not whole 128-column rotation blocks): there the aliasing call returns
 * LRQ_ERR_UNSUPPORTED. */

/* dx = dy * s(x)(1 + x(1 - s(x))), s = sigmoid, x = decode(t), fused.
 * Replaces triton_silu_backward_fuse_extraction (extraction_fuse_silu_backward.py:192-216). */
int lrq_silu_bwd(const lrq_tensors* t, const void* dy, int64_t lddy, void* dx, int64_t lddx, void* stream);

/* dx = tanh-GELU'(x) * dy, x = decode(t), fused (gelu_backward.py:14-21 formula; the reference
 * has only the uncompressed triton_gelu_backward, gelu_backward.py:73-88). */
int lrq_gelu_bwd(const lrq_tensors* t, const void* dy, int64_t lddy, void* dx, int64_t lddx, void* stream);

/* out = decode(t) * y elementwise.
 * Replaces triton_hadamard_fuse_extraction (extraction_fuse_hadamard.py:185-209). */
int lrq_mul(const lrq_tensors* t, const void* y, int64_t ldy, void* out, int64_t ldo, void* stream);

/* ds = p * (dp - rowsum(dp * p)), p = decode(t) (rows = softmax rows), fused with the row sum
 * (softmax_backward.py:6-7 formula; the reference has only the uncompressed
 * triton_softmax_backward, softmax_backward.py:45-61). */
int lrq_softmax_bwd(const lrq_tensors* t, const void* dp, int64_t lddp, void* ds, int64_t ldds,
                    void* stream);

/* out[rows, n_out] = decode(t) @ a[hidden, n_out] (a bf16 row-major), fp32 accumulate;
 * out is fp32 when out_fp32 != 0, else bf16.
 * Replaces triton_matmul_decompress (extraction_fuse_matmul.py:224-249). */
int lrq_dequant_gemm(const lrq_tensors* t, const void* a, int32_t n_out, void* out, int64_t ldo,
                     int32_t out_fp32, void* stream);

/* out[hidden, n_out] = decode(t)^T @ g[rows, n_out] (g bf16 row-major, ld ldg a multiple of 4,
 * 8-byte aligned), fp32 accumulate, decode(t) rounded to bf16 as lrq_decode returns it; out is
 * fp32 when out_fp32 != 0, else bf16.  n_out is 16 or 32.  Outlier channels: their output rows
 * come from the side columns, as the decode returns them.  The rotated format: decode(t) is the
 * rotated decode's bf16 result (hidden/NP a multiple of 128).  This is the LoRA factor gradient dA = x^T (dy B^T) of compute_lora_gradient
 * (low_rank_system_profile_forward.py:14-18, `x.mT @ (dy @ b.mT)`) read from the codes: a
 * reduction over the rows.  The rows are split into groups whose fp32 partials [hidden, n_out]
 * go to `workspace` (16-byte aligned, at least lrq_dequant_gemm_t_workspace(t, n_out) bytes),
 * then summed in group order: results depend only on the shapes, not on timing.  rows == 0
 * writes zeros. */
int lrq_dequant_gemm_t(const lrq_tensors* t, const void* g, int64_t ldg, int32_t n_out, void* out,
                       int64_t ldo, int32_t out_fp32, void* workspace, int64_t workspace_bytes,
                       void* stream);

/* Workspace bytes lrq_dequant_gemm_t needs for `t` and n_out (>= 0), or a negative LRQ_ERR_*.
 * Host only: no HIP call. */
int64_t lrq_dequant_gemm_t_workspace(const lrq_tensors* t, int32_t n_out);

/* Both LoRA factor-gradient products that read the saved activation, in one pass over its
 * codes: xa[rows, n_out] = decode(t) a (a bf16 [hidden, n_out], row stride lda) — the x A whose
 * transpose times dy is dB — and da[hidden, n_out] = decode(t)^T g (g bf16 [rows, n_out], row
 * stride ldg, 8-byte aligned) — dA = x^T (dy B^T); compute_lora_gradient
 * (low_rank_system_profile_forward.py:14-18, `(x @ a).mT @ dy` and `x.mT @ (dy @ b.mT)`).  Same
 * results as lrq_dequant_gemm (xa) and lrq_dequant_gemm_t (da) up to the order of the fp32
 * additions: decode(t) rounded to bf16 as lrq_decode returns it, fp32 accumulate; each output
 * fp32 when its *_fp32 flag is non-zero (16-byte aligned rows of a multiple of 4 elements), else
 * bf16 (8-byte aligned).  int4 / group 64 / rank 16, n_out 16, a multiple of 4 units (512
 * columns) per row, no outlier channels, no rotated format (else LRQ_ERR_UNSUPPORTED: use the two
 * entry points).  The fp32 partials of column and row groups go to `workspace` (16-byte
 * aligned, lrq_lora_grads_workspace(t, n_out) bytes) and are summed in group order, so results
 * depend only on the shapes.  rows == 0 writes zeros to da. */
int lrq_lora_grads(const lrq_tensors* t, const void* a, int64_t lda, const void* g, int64_t ldg, int32_t n_out,
                   void* xa, int64_t ldxa, int32_t xa_fp32, void* da, int64_t ldda, int32_t da_fp32,
                   void* workspace, int64_t workspace_bytes, void* stream);

/* Workspace bytes lrq_lora_grads needs for `t` and n_out (>= 0), or a negative LRQ_ERR_*.
 * Host only: no HIP call. */
int64_t lrq_lora_grads_workspace(const lrq_tensors* t, int32_t n_out);

/* Largest workspace lrq_dequant_gemm_t_noalloc can serve from its own scratch (bytes). */
#define LRQ_GEMM_T_SCRATCH_BYTES (16 * 1024 * 1024)

/* Allocation-free form of lrq_dequant_gemm_t.  No counterpart in the reference: it is for
 * callers that cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc).  Same arguments, kernels and results as
 * lrq_dequant_gemm_t, without the workspace: the row-group partials go to a scratch array of
 * LRQ_GEMM_T_SCRATCH_BYTES that the library keeps in device memory, one per GPU it runs on,
 * held until the process ends.  The call allocates nothing.  Shapes whose
 * lrq_dequant_gemm_t_workspace(t, n_out) exceeds the scratch return LRQ_ERR_WORKSPACE (checked
 * on the host before any HIP call).  Every call on one GPU shares that GPU's scratch, and the
 * scratch keeps the last call's partials: calls that overlap on one GPU (different streams or
 * threads without ordering between them) race; calls ordered on one stream do not. */
int lrq_dequant_gemm_t_noalloc(const lrq_tensors* t, const void* g, int64_t ldg, int32_t n_out, void* out,
                               int64_t ldo, int32_t out_fp32, void* stream);

/* colmax[c] = max_r |x[r, c]| (fp32).  First half of the outlier-channel split
 * (no reference counterpart; the reference's channel split takes caller indices,
 * extraction_outlier_channel.py:11-14). */
int lrq_colmax(const void* x, int64_t ldx, int64_t rows, int64_t hidden, float* colmax, void* stream);

/* idx = the k columns with the largest colmax, ascending; ties toward the lower index. */
int lrq_topk(const float* colmax, int64_t hidden, int32_t k, int32_t* idx, void* stream);

/* dst[cols, rows] = src[rows, cols]^T for bf16 (builds Vt from V, and V-layout from the
 * reference's r[K, N] factor). */
int lrq_transpose_bf16(const void* src, int64_t rows, int64_t cols, void* dst, void* stream);

/* y = bf16(WHT128(x)) per 128-column block of every row: the normalised Walsh-Hadamard
 * rotation (its own inverse), sums accumulated on MFMA in four 32-column steps.  x, y:
 * bf16 [rows, hidden] with 16-byte aligned rows, hidden % 128 == 0; y may equal x (in place).
 * No reference function (north-star config 4). */
int lrq_wht128(const void* x, int64_t ldx, int64_t rows, int64_t hidden, void* y, int64_t ldy, void* stream);

/* ------------------------------------------------------------------ legacy mode
 * The reference's own formulation: caller-supplied factors l[M, K] (bf16) and r as
 * rt[N, K] (= r^T, bf16), per-column symmetric scale s[S, N] (bf16; batch b uses row
 * b % S), threshold outliers kept as a dense bf16 tensor, row-planar packing.  x is
 * [B, M, N] bf16 with leading dims (ldx_b, ldx_m); row-major in N.  Arithmetic follows
 * the reference's torch forms, bf16 rounding after each op. */

/* Replaces low_rank_addition_fuse_compression_quantization
 * (low_rank_extraction_fuse_compression_quantization.py:118-150; torch form :153-171).
 * o[B, M, N] receives the dense outliers (bf16), q[B, M, N*bits/8] the codes. */
int lrq_legacy_encode(const void* l, const void* rt, int32_t K, const void* x, int64_t B, int64_t M,
                      int64_t N, int64_t ldx_b, int64_t ldx_m, const void* s, int64_t s_rows,
                      int32_t bits, float outlier, void* o, void* q, void* stream);

/* Replaces low_rank_addition_fuse_decompression_dequantization
 * (low_rank_extraction_fuse_decompression_dequantization.py:116-152; torch form :155-165).
 * o may be NULL (no outliers).  out[B, M, N] bf16. */
int lrq_legacy_decode(const void* l, const void* rt, int32_t K, const void* q, const void* o,
                      const void* s, int64_t s_rows, int64_t B, int64_t M, int64_t N, int32_t bits,
                      void* out, void* stream);

/* Dense -> COO compaction of the legacy outliers o[B, M, N] (bf16, contiguous): the coalesced COO
 * tensor o.to_sparse() builds (low_rank_extraction_fuse_compression_quantization.py:149), on the
 * device and without a host synchronisation.  Entries (bf16 bits not +-0) in row-major order:
 * indices int64 [3, ld_idx] (rows b, m, n; entry e in column e), values bf16 [cap]; entries at
 * positions >= cap are not written, and *nnz (int64, device) is the full count, so nnz > cap
 * tells the caller to grow the buffers and call again.  piece_ptr int64 [B*M*ceil(N/64) + 1]
 * receives the first entry of every 64-column piece of a row (the last element is nnz): the
 * lookup lrq_legacy_decode_coo reads.  workspace: lrq_coo_workspace(B, M, N) bytes, 8-aligned. */
int lrq_coo_compact(const void* o, int64_t B, int64_t M, int64_t N, int64_t* indices, int64_t ld_idx,
                    void* values, int64_t cap, int64_t* nnz, int64_t* piece_ptr, void* workspace,
                    int64_t workspace_bytes, void* stream);

/* Workspace bytes of lrq_coo_compact (>= 0), or a negative LRQ_ERR_*.  Host only. */
int64_t lrq_coo_workspace(int64_t B, int64_t M, int64_t N);

/* lrq_legacy_encode followed by lrq_coo_compact of its outliers: the reference's encode plus
 * o.to_sparse() (low_rank_extraction_fuse_compression_quantization.py:118-150), without its host
 * synchronisation; codes q, indices, values, *nnz and piece_ptr as the two calls give them.  On the
 * encode's vectorised path (bits * N % 512 == 0, 16-byte aligned operands, outlier >= 0) the encode
 * stages each 64-column piece's count and first two entries in piece_ptr as it quantises, and
 * writes a piece's dense values to o only when it has more entries than that; the compaction then
 * reads the staged pieces and only those dense ones.  o [B, M, N] bf16 is therefore working memory:
 * its contents on return are unspecified (the two calls' dense outliers come from
 * lrq_legacy_encode).  Other shapes run the two calls. */
int lrq_legacy_encode_coo(const void* l, const void* rt, int32_t K, const void* x, int64_t B, int64_t M,
                          int64_t N, int64_t ldx_b, int64_t ldx_m, const void* s, int64_t s_rows,
                          int32_t bits, float outlier, void* o, void* q, int64_t* indices, int64_t ld_idx,
                          void* values, int64_t cap, int64_t* nnz, int64_t* piece_ptr, void* workspace,
                          int64_t workspace_bytes, void* stream);

/* lrq_legacy_decode with the outliers as COO pieces instead of a dense tensor: piece_ptr as
 * lrq_coo_compact writes it, cols = the entries' column indices (int64, row 2 of its indices),
 * vals = their bf16 values, n_entries = how many entries cols / vals hold (reads are clamped to
 * it: entries a too-small compaction dropped are missing from the result, so check nnz first).  Each element adds the outlier of its own column, if any, at the same
 * point of the torch form as the dense decode: the two give the same bits.  Replaces the
 * o.to_dense() of low_rank_addition_fuse_decompression_dequantization
 * (low_rank_extraction_fuse_decompression_dequantization.py:136). */
int lrq_legacy_decode_coo(const void* l, const void* rt, int32_t K, const void* q, const int64_t* piece_ptr,
                          const int64_t* cols, const void* vals, int64_t n_entries, const void* s,
                          int64_t s_rows, int64_t B, int64_t M, int64_t N, int32_t bits, void* out,
                          void* stream);

/* *out = the k-th smallest (1-based) of |bf16(x - bf16(l @ r))| over one [M, N] slice of x (rows
 * ldx_m apart), as fp32 on the device: the outlier threshold
 * torch.kthvalue((x[0] - L_x @ R_x).flatten().abs().to(torch.float32), k) of
 * low_rank_system_profile_forward.py:45 (k = numel * 0.99 there), with the residual computed as
 * lrq_legacy_encode computes it.  Two histogram passes over the 15-bit magnitudes; M * N < 2^32,
 * 1 <= k <= M * N.  workspace >= 2048 bytes, 16-aligned. */
int lrq_legacy_kth_residual(const void* l, const void* rt, int32_t K, const void* x, int64_t M, int64_t N,
                            int64_t ldx_m, int64_t k, float* out, void* workspace, int64_t workspace_bytes,
                            void* stream);

/* Fused legacy consumers (no outliers): op = 0 store x_hat, 1 SiLU backward with y as dy
 * (extraction_fuse_silu_backward.py:192-216), 2 elementwise product with y
 * (extraction_fuse_hadamard.py:185-209).  y, out: [B, M, N] bf16 contiguous. */
int lrq_legacy_fused(const void* l, const void* rt, int32_t K, const void* q, const void* s,
                     int64_t s_rows, int64_t B, int64_t M, int64_t N, int32_t bits, int32_t op,
                     const void* y, void* out, void* stream);

/* Fused legacy dequant-GEMM (no outliers): out[b, m, c] = bf16(sum_n x_hat[b, m, n] * y[b, n, c]),
 * fp32 sums, x_hat the decode's value computed in registers and never stored.  y: bf16
 * [B, N, ldy] (batch stride N * ldy), out: bf16 [B, M, ldo] (batch stride M * ldo), c < n_out.
 * Replaces triton_matmul_decompress (extraction_fuse_matmul.py:224-249, kernel :151-221; torch
 * form torch_matmul :5-6 of the decoded activation). */
int lrq_legacy_dequant_gemm(const void* l, const void* rt, int32_t K, const void* q, const void* s,
                            int64_t s_rows, int64_t B, int64_t M, int64_t N, int32_t bits, const void* y,
                            int64_t ldy, int32_t n_out, void* out, int64_t ldo, void* stream);

/* out = x + l @ r (bf16 semantics of torch_low_rank_addition).
 * Replaces low_rank_addition (low_rank_extraction_speed.py:77-103). */
int lrq_lowrank_add(const void* l, const void* rt, int32_t K, const void* x, int64_t B, int64_t M,
                    int64_t N, void* out, void* stream);

/* ------------------------------------------------------------------ dense consumers
 * Uncompressed elementwise kernels over n contiguous bf16 elements.
 * op: 0 SiLU bwd (triton_silu_backward, silu_backward.py:54-69),
 *     1 GELU bwd (triton_gelu_backward, gelu_backward.py:73-88),
 *     2 product  (triton_hadamard, extraction_fuse_hadamard.py:62-73). */
int lrq_dense_elementwise(int32_t op, const void* x, const void* y, void* out, int64_t n, void* stream);

/* ds = y * (g - rowsum(g * y)) over rows of length n_cols, contiguous bf16.
 * Replaces triton_softmax_backward (softmax_backward.py:45-61). */
int lrq_dense_softmax_bwd(const void* y, const void* g, void* out, int64_t rows, int64_t n_cols,
                          void* stream);

/* outlier = x * (|x| > bf16(threshold)), rest = x - outlier over n contiguous bf16.
 * Replaces torch_extract_unstructured (extraction_outlier_channel.py:5-8); the caller makes
 * the sparse COO tensor of outlier, as the reference does. */
int lrq_threshold_split(const void* x, int64_t n, float threshold, void* outlier, void* rest, void* stream);

/* out[b, i, :] = x[b, idx[i], :] and x[b, idx[i], :] = 0 (in place) for x [B, M, N] bf16
 * contiguous, k distinct indices along dim 1 (the reference's axis).
 * Replaces torch_extract_channel (extraction_outlier_channel.py:11-14). */
int lrq_gather_rows_zero(void* x, int64_t B, int64_t M, int64_t N, const int32_t* idx, int32_t k, void* out,
                         void* stream);

/* ------------------------------------------------------------------ misc */
const char* lrq_status_string(int status);
int32_t lrq_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* LRQ_H */
