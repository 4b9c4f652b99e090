"""GPU parity of the reference-format ("legacy") operators and the dense consumers.

Each reference entry point (legacy.py) runs on the HIP kernels and is compared with the CPU
restatement of the reference's torch form (oracle/lrq_oracle.py legacy_* functions).  The
torch forms round to bf16 after every op; the kernels reproduce those roundings, and l @ r
is the fp32 rounding of the exact sum in both, so codes, outliers and bf16 outputs are
expected to match bit for bit (the assertion allows the north-star tie budget of 1e-4).
Shapes cover both kernel paths: the MFMA path (every plane a multiple of 64 columns,
16-byte aligned operands) and the scalar path (the reference's 32 x 32 smoke shape, odd
widths, unaligned row strides), K below 16 and between 16 and 32 (zero-padded, R14),
batch-shared and per-batch scales, 1/2/4/8-bit codes.
"""

import ctypes
import importlib

import numpy as np
import pytest
import torch

import oracle as O
from parity import TIE_BUDGET, assert_fp_close, bits16, from_bits

pytestmark = pytest.mark.gpu


def _inputs(seed, B, M, N, K, s_rows, scale_lo=0.05, scale_hi=0.4, outlier_cols=4):
    g = torch.Generator().manual_seed(seed)
    l = (torch.randn(M, K, generator=g) * 0.5).to(torch.bfloat16)
    r = (torch.randn(K, N, generator=g) * 0.5).to(torch.bfloat16)
    x = torch.randn(B, M, N, generator=g)
    cols = torch.randperm(N, generator=g)[:outlier_cols]
    x[:, :, cols] *= 12.0
    x = x.to(torch.bfloat16)
    s = (scale_lo + (scale_hi - scale_lo) * torch.rand(s_rows, N, generator=g)).to(torch.bfloat16)
    return l, r, x, s


def _frac_mismatch(a: np.ndarray, b: np.ndarray) -> float:
    return float((a != b).sum()) / max(1, a.size)


CASES = [
    # (B, M, N, K, bits, s_rows, tau) — path noted
    (1, 32, 32, 16, 4, 1, 5.0),      # reference smoke shape: scalar path
    (2, 100, 1024, 16, 4, 2, 5.0),   # MFMA, per-batch scales, ragged rows
    (1, 64, 2048, 32, 8, 1, 5.0),    # MFMA, K = 32
    (1, 48, 1024, 8, 2, 1, 4.0),     # MFMA, K = 8 padded to 16
    (1, 40, 1024, 16, 1, 1, 12.0),   # MFMA, 1-bit (8 planes), tau = 12 as the encode speed test
    (3, 17, 96, 20, 4, 3, 5.0),      # scalar, K = 20 padded to 32
]


@pytest.mark.parametrize("bits", [1, 2, 4, 8])
def test_legacy_encode_extreme_scales(pkg, dev, bits):
    """Scales outside [2^-100, 2^100] (here 2^-110 and 2^105, in a few columns of some units)
    send their workgroups to the IEEE division; the other units take the reciprocal form.
    Codes and outliers equal the oracle's on both."""
    B, M, N, K, tau = 1, 64, 2048, 16, 5.0
    l, r, x, s = _inputs(4242 + bits, B, M, N, K, 1)
    s = s.float()
    s[0, 3] = 2.0 ** -110
    s[0, 700] = 2.0 ** 105
    s[0, N - 1] = -(2.0 ** -110)
    s = s.to(torch.bfloat16)
    lb, rb, xb, sb = bits16(l), bits16(r), bits16(x), bits16(s)
    o_sp, q = pkg.low_rank_addition_fuse_compression_quantization(l.to(dev), r.to(dev), x.to(dev), s.to(dev),
                                                                  quantize_bit=bits, outlier=tau)
    torch.cuda.synchronize()
    o_ref, q_ref = O.legacy_encode(lb, rb, xb, sb, bits, tau)
    qg = q.cpu().numpy()
    assert _frac_mismatch(qg, q_ref) <= TIE_BUDGET
    og = bits16(o_sp.to_dense())
    nz = (O.bf16_to_f32(o_ref) != 0) | (O.bf16_to_f32(og) != 0)
    assert _frac_mismatch(og[nz], o_ref[nz]) <= TIE_BUDGET


@pytest.mark.parametrize("B,M,N,K,bits,s_rows,tau", CASES)
def test_legacy_encode_decode(pkg, dev, B, M, N, K, bits, s_rows, tau):
    l, r, x, s = _inputs(1000 + N + bits, B, M, N, K, s_rows)
    lb, rb, xb, sb = bits16(l), bits16(r), bits16(x), bits16(s)
    o_sp, q = pkg.low_rank_addition_fuse_compression_quantization(l.to(dev), r.to(dev), x.to(dev), s.to(dev),
                                                                  quantize_bit=bits, outlier=tau)
    torch.cuda.synchronize()
    assert o_sp.is_sparse
    o_ref, q_ref = O.legacy_encode(lb, rb, xb, sb, bits, tau)
    qg = q.cpu().numpy()
    assert qg.shape == q_ref.shape
    fq = _frac_mismatch(qg, q_ref)
    assert fq <= TIE_BUDGET, f"code bytes differ: {fq}"
    og = bits16(o_sp.to_dense())
    # outliers: values equal; the sign of non-outlier zeros is not part of the format
    nz = (O.bf16_to_f32(o_ref) != 0) | (O.bf16_to_f32(og) != 0)
    assert _frac_mismatch(og[nz], o_ref[nz]) <= TIE_BUDGET
    assert int(nz.sum()) > 0, "test data should contain outliers"

    # decode of the oracle's own (q, o): bf16 bit parity
    xh = pkg.low_rank_addition_fuse_decompression_dequantization(
        l.to(dev), r.to(dev), torch.from_numpy(q_ref).to(dev), from_bits(o_ref, dev), s.to(dev), quantize_bit=bits)
    xh_ref = O.legacy_decode(lb, rb, q_ref, o_ref, sb, bits)
    assert _frac_mismatch(bits16(xh), xh_ref) <= TIE_BUDGET

    # round trip through the device's own encode == the unpacked naive round trip (R5)
    xh2 = pkg.low_rank_addition_fuse_decompression_dequantization(l.to(dev), r.to(dev), q, o_sp, s.to(dev),
                                                                  quantize_bit=bits)
    naive = O.naive_roundtrip(lb, rb, xb, sb, bits, tau)
    assert _frac_mismatch(bits16(xh2), naive) <= TIE_BUDGET

    # decode without outliers
    xh3 = pkg.low_rank_addition_fuse_decompression_dequantization(l.to(dev), r.to(dev), q, None, s.to(dev),
                                                                  quantize_bit=bits)
    assert _frac_mismatch(bits16(xh3), O.legacy_decode(lb, rb, qg, None, sb, bits)) <= TIE_BUDGET


def test_legacy_encode_strided_input(pkg, dev):
    """x rows with a padded stride (the reference passes x's strides to its kernel): an
    8-aligned stride stays on the MFMA path, an odd one takes the scalar path."""
    B, M, N, K, bits = 2, 40, 1024, 16, 4
    l, r, x, s = _inputs(77, B, M, N, K, 1)
    for pad in (8, 3):
        wide = torch.zeros(B, M, N + pad, dtype=torch.bfloat16)
        wide[:, :, :N] = x
        xs = wide.to(dev)[:, :, :N]
        assert xs.stride(1) == N + pad
        o_sp, q = pkg.low_rank_addition_fuse_compression_quantization(l.to(dev), r.to(dev), xs, s.to(dev),
                                                                      quantize_bit=bits)
        o_ref, q_ref = O.legacy_encode(bits16(l), bits16(r), bits16(x), bits16(s), bits, 5.0)
        assert _frac_mismatch(q.cpu().numpy(), q_ref) <= TIE_BUDGET, f"pad {pad}"


FUSED = [
    (1, 64, 1024, 16, 2),   # the fused wrappers' default 2-bit codes, MFMA path
    (2, 33, 1024, 16, 4),   # ragged rows, batch 2
    (1, 32, 32, 16, 2),     # scalar path
]


@pytest.mark.parametrize("B,M,N,K,bits", FUSED)
def test_legacy_fused_consumers(pkg, dev, B, M, N, K, bits):
    l, r, x, s = _inputs(5000 + N, B, M, N, K, 1, outlier_cols=0)
    lb, rb, xb, sb = bits16(l), bits16(r), bits16(x), bits16(s)
    _, q_ref = O.legacy_encode(lb, rb, xb, sb, bits, 1e9)
    xh = O.bf16_to_f32(O.legacy_decode(lb, rb, q_ref, None, sb, bits))
    g = torch.Generator().manual_seed(99)
    dy = (torch.randn(B, M, N, generator=g) * 0.02).to(torch.bfloat16)
    yb = bits16(dy)
    yf = O.bf16_to_f32(yb)
    q = torch.from_numpy(q_ref).to(dev)
    args = (l.to(dev), r.to(dev), q, s.to(dev), dy.to(dev))
    out = pkg.triton_silu_backward_fuse_extraction(*args, quantize_bit=bits)
    assert_fp_close(bits16(out), O.silu_bwd(xh, yf), "legacy fused SiLU bwd")
    out = pkg.triton_silu_backward_add_extraction(*args, quantize_bit=bits)
    assert_fp_close(bits16(out), O.silu_bwd(xh, yf), "legacy unfused SiLU bwd")
    out = pkg.triton_hadamard_fuse_extraction(*args, quantize_bit=bits)
    assert _frac_mismatch(bits16(out), O.round_out(O.mul(xh, yf))) <= TIE_BUDGET
    out = pkg.triton_hadamard_add_extraction(*args, quantize_bit=bits)
    assert _frac_mismatch(bits16(out), O.round_out(O.mul(xh, yf))) <= TIE_BUDGET
    # dequant-matmul (R12, legacy format): x_hat @ y with y [B, N, 32]
    yk = (torch.randn(B, N, 32, generator=g) * 0.1).to(torch.bfloat16)
    mm = pkg.triton_matmul_decompress(q, l.to(dev), r.to(dev), s.to(dev), yk.to(dev), quantize_bit=bits)
    ref = np.stack([O.gemm(xh[b], O.bf16_to_f32(bits16(yk[b]))) for b in range(B)])
    assert_fp_close(bits16(mm), ref, "legacy dequant matmul")


GEMM = [
    # (B, M, N, K, bits, n, s_rows) — the reference bench's y [B, N, 32] and 2-bit codes first
    (2, 100, 1024, 32, 2, 32, 1),   # MFMA, ragged rows, K = 32, batch 2
    (3, 64, 2048, 16, 1, 16, 3),    # 1-bit (8 planes), per-batch scales
    (2, 48, 1024, 8, 4, 48, 1),     # K = 8 padded to 16; n = 48 = a 32- and a 16-column chunk
    (1, 300, 1024, 20, 8, 20, 1),   # 8-bit, K = 20 padded to 32, n = 20 padded to 32
    (2, 17, 96, 16, 2, 32, 2),      # scalar path (planes of 24 columns)
    (1, 32, 32, 16, 4, 7, 1),       # scalar path, the reference smoke shape, n = 7
]


@pytest.mark.parametrize("B,M,N,K,bits,n,s_rows", GEMM)
def test_legacy_dequant_gemm(pkg, dev, B, M, N, K, bits, n, s_rows):
    """triton_matmul_decompress (R12, legacy format) in one kernel: x_hat @ y against the
    float64 product of the oracle's decoded x_hat, at the north-star floating-point bars."""
    l, r, x, s = _inputs(7100 + N + bits, B, M, N, K, s_rows, outlier_cols=0)
    lb, rb, xb, sb = bits16(l), bits16(r), bits16(x), bits16(s)
    _, q_ref = O.legacy_encode(lb, rb, xb, sb, bits, 1e9)
    xh = O.bf16_to_f32(O.legacy_decode(lb, rb, q_ref, None, sb, bits))
    g = torch.Generator().manual_seed(71 + n)
    y = (torch.randn(B, N, n, generator=g) * 0.1).to(torch.bfloat16)
    q = torch.from_numpy(q_ref).to(dev)
    out = pkg.triton_matmul_decompress(q, l.to(dev), r.to(dev), s.to(dev), y.to(dev), quantize_bit=bits)
    assert tuple(out.shape) == (B, M, n) and out.dtype == torch.bfloat16
    ref = np.stack([O.gemm(xh[b], O.bf16_to_f32(bits16(y[b]))) for b in range(B)])
    assert_fp_close(bits16(out), ref, f"legacy dequant-GEMM {bits}-bit K={K} n={n}")


def test_legacy_dequant_gemm_strided_y_and_empty(pkg, dev):
    """A non-contiguous y (a transposed view) gives the same bits as its contiguous copy, and
    zero rows or zero output columns return empty results."""
    B, M, N, K, bits = 2, 64, 1024, 16, 2
    l, r, x, s = _inputs(7300, B, M, N, K, 1, outlier_cols=0)
    _, q_ref = O.legacy_encode(bits16(l), bits16(r), bits16(x), bits16(s), bits, 1e9)
    q = torch.from_numpy(q_ref).to(dev)
    g = torch.Generator().manual_seed(73)
    yt = (torch.randn(B, 32, N, generator=g) * 0.1).to(torch.bfloat16).to(dev)
    a = pkg.triton_matmul_decompress(q, l.to(dev), r.to(dev), s.to(dev), yt.transpose(1, 2), quantize_bit=bits)
    b = pkg.triton_matmul_decompress(q, l.to(dev), r.to(dev), s.to(dev), yt.transpose(1, 2).contiguous(),
                                     quantize_bit=bits)
    assert torch.equal(a, b)
    e = pkg.triton_matmul_decompress(q, l.to(dev), r.to(dev), s.to(dev), yt.transpose(1, 2)[..., :0],
                                     quantize_bit=bits)
    assert tuple(e.shape) == (B, M, 0)


@pytest.mark.parametrize("B,M,N,K", [(2, 100, 1024, 16), (1, 32, 32, 8), (1, 16, 96, 32)])
def test_low_rank_addition(pkg, dev, B, M, N, K):
    l, r, x, _ = _inputs(300 + N, B, M, N, K, 1)
    out = pkg.low_rank_addition(l.to(dev), r.to(dev), x.to(dev))
    ref = O.lowrank_add(bits16(l), bits16(r), bits16(x))
    assert _frac_mismatch(bits16(out), ref) <= TIE_BUDGET


@pytest.mark.parametrize("shape", [(2, 64, 1024), (1, 7, 333)])
def test_dense_elementwise(pkg, dev, shape):
    g = torch.Generator().manual_seed(11)
    x = (torch.randn(*shape, generator=g) * 2).to(torch.bfloat16)
    y = (torch.randn(*shape, generator=g) * 0.02).to(torch.bfloat16)
    xf, yf = O.bf16_to_f32(bits16(x)), O.bf16_to_f32(bits16(y))
    assert_fp_close(bits16(pkg.triton_silu_backward(x.to(dev), y.to(dev))), O.silu_bwd(xf, yf), "dense SiLU bwd")
    assert_fp_close(bits16(pkg.triton_gelu_backward(x.to(dev), y.to(dev))), O.gelu_bwd(xf, yf), "dense GELU bwd")
    assert _frac_mismatch(bits16(pkg.triton_hadamard(x.to(dev), y.to(dev))), O.round_out(O.mul(xf, yf))) == 0


@pytest.mark.parametrize("shape", [(2, 4, 64, 64), (1, 2, 8, 2048), (1, 1, 5, 2050), (1, 1, 3, 10000)])
def test_dense_softmax_bwd(pkg, dev, shape):
    g = torch.Generator().manual_seed(12)
    logits = torch.randn(*shape, generator=g) / np.sqrt(128)
    p = torch.softmax(logits, dim=-1).to(torch.bfloat16)
    dp = (torch.randn(*shape, generator=g) * 0.02).to(torch.bfloat16)
    pf, dpf = O.bf16_to_f32(bits16(p)), O.bf16_to_f32(bits16(dp))
    out = pkg.triton_softmax_backward(p.to(dev), dp.to(dev))
    assert_fp_close(bits16(out), O.softmax_bwd(pf, dpf), "dense softmax bwd", max_abs=1e-3)


def test_outlier_extraction_forms(pkg, dev):
    """torch_extract_unstructured / torch_extract_channel (extraction_outlier_channel.py:5-14)."""
    g = torch.Generator().manual_seed(13)
    x = (torch.randn(2, 64, 96, generator=g) * 2).to(torch.bfloat16)
    xb = bits16(x)
    xf = O.bf16_to_f32(xb)
    thr = torch.tensor(2.3)  # as the reference passes a kthvalue result
    o_sp, rest = pkg.torch_extract_unstructured(x.to(dev), thr.to(dev))
    tau = O.bf16_to_f32(O.bf16_round(np.float32(2.3)))
    mask = np.abs(xf) > tau
    assert np.array_equal(bits16(o_sp.to_dense()), np.where(mask, xb, 0).astype(np.uint16))
    assert np.array_equal(bits16(rest), np.where(mask, 0, xb).astype(np.uint16))
    idx = [3, 10, 40, 63]
    xd = x.to(dev).contiguous()
    out, x2 = pkg.torch_extract_channel(xd, idx)
    assert x2.data_ptr() == xd.data_ptr()  # in place, like the reference
    assert np.array_equal(bits16(out), xb[:, idx, :])
    ref = xb.copy()
    ref[:, idx, :] = 0
    assert np.array_equal(bits16(x2), ref)


# ------------------------------------------------------------------ outliers as COO on the GPU
COO_SHAPES = [(2, 100, 1024), (1, 33, 70), (64, 4096), (5000,), (3, 7, 96), (2, 3, 4, 64)]


def _sparse_dense(shape, seed, keep=0.03):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(shape, generator=g) * 8
    x = torch.where(torch.rand(shape, generator=g) < 1 - keep, torch.zeros(shape), x)
    x.view(-1)[::11] = -0.0  # negative zeros are not entries
    return x.to(torch.bfloat16)


@pytest.mark.parametrize("shape", COO_SHAPES)
def test_coo_compaction_is_to_sparse(pkg, dev, shape):
    """The GPU compaction gives o.to_sparse() exactly (indices, value bits, coalesced), and piece
    pointers = the first entry of every 64-column piece of a row."""
    print(f"[coo] shape={shape}", flush=True)
    x = _sparse_dense(shape, sum(shape))
    idx_ref, val_ref = O.to_coo(bits16(x))
    sp = pkg.legacy._to_sparse(x.to(dev))
    torch.cuda.synchronize()
    assert sp.is_sparse and sp.is_coalesced() and tuple(sp.shape) == shape
    assert np.array_equal(sp.indices().cpu().numpy(), idx_ref)
    assert np.array_equal(bits16(sp.values()), val_ref)
    if len(shape) <= 3:
        c = pkg.compact_outliers(x.to(dev))
        B, M, N = (1,) * (3 - len(shape)) + shape
        full = np.zeros((3, idx_ref.shape[1]), np.int64)
        full[3 - len(shape):] = idx_ref
        npc = (N + 63) // 64
        pid = (full[0] * M + full[1]) * npc + full[2] // 64
        ptr_ref = np.searchsorted(pid, np.arange(B * M * npc + 1))
        assert np.array_equal(c.piece_ptr.cpu().numpy(), ptr_ref)
        assert int(c.nnz.item()) == idx_ref.shape[1]


def test_coo_capacity_overflow(pkg, dev):
    """Fewer slots than entries: the first `cap` entries are written, nnz is the full count and
    to_sparse refuses."""
    x = _sparse_dense((40, 1024), 9, keep=0.1)
    idx_ref, val_ref = O.to_coo(bits16(x))
    n = idx_ref.shape[1]
    c = pkg.compact_outliers(x.to(dev), capacity=n // 3)
    torch.cuda.synchronize()
    assert int(c.nnz.item()) == n
    k = n // 3
    assert np.array_equal(c.indices[1:, :k].cpu().numpy(), idx_ref[:, :k])
    assert np.array_equal(bits16(c.values[:k]), val_ref[:k])
    with pytest.raises(RuntimeError):
        c.to_sparse()


@pytest.mark.parametrize("B,M,N,K,bits,s_rows,tau", [CASES[0], CASES[1], CASES[2], CASES[5]])
def test_legacy_decode_coo_is_dense_decode(pkg, dev, B, M, N, K, bits, s_rows, tau):
    """The decode that reads COO pieces gives the dense decode's bits, for the encode's own
    LegacyOutliers (no host synchronisation) and for a torch sparse tensor."""
    print(f"[coo decode] B={B} M={M} N={N} K={K} bits={bits}", flush=True)
    l, r, x, s = _inputs(2000 + N + bits, B, M, N, K, s_rows)
    ld, rd, xd, sd = l.to(dev), r.to(dev), x.to(dev), s.to(dev)
    oc, q = pkg.legacy_encode_coo(ld, rd, xd, sd, quantize_bit=bits, outlier=tau)
    o_sp, q2 = pkg.low_rank_addition_fuse_compression_quantization(ld, rd, xd, sd, quantize_bit=bits, outlier=tau)
    assert torch.equal(q, q2)
    dense = o_sp.to_dense()
    a = pkg.low_rank_addition_fuse_decompression_dequantization(ld, rd, q, oc, sd, quantize_bit=bits)
    b = pkg.low_rank_addition_fuse_decompression_dequantization(ld, rd, q, o_sp, sd, quantize_bit=bits)
    c = pkg.low_rank_addition_fuse_decompression_dequantization(ld, rd, q, dense, sd, quantize_bit=bits)
    torch.cuda.synchronize()
    assert int(oc.nnz.item()) == o_sp._nnz() > 0
    assert torch.equal(a, c) and torch.equal(b, c)
    o_ref, _ = O.legacy_encode(bits16(l), bits16(r), bits16(x), bits16(s), bits, tau)
    xh_ref = O.legacy_decode(bits16(l), bits16(r), q.cpu().numpy(), bits16(dense), bits16(s), bits)
    assert _frac_mismatch(bits16(a), xh_ref) <= TIE_BUDGET


@pytest.mark.parametrize("B,M,N,K,bits,s_rows,tau", [CASES[0], CASES[1], CASES[2], CASES[5],
                                                    (2, 37, 512, 16, 1, 2, 1.5), (1, 80, 1024, 16, 2, 1, 0.5)])
def test_legacy_encode_coo_is_encode_then_compact(pkg, dev, B, M, N, K, bits, s_rows, tau):
    """lrq_legacy_encode_coo (the encode staging each piece's count and first entries, then chunk
    totals, chunk scan and scatter) gives exactly what lrq_legacy_encode followed by
    lrq_coo_compact gives: codes, COO indices and values, entry count and piece pointers (dense-ish
    outliers with a low threshold included: pieces read from their dense values)."""
    print(f"[encode_coo] B={B} M={M} N={N} K={K} bits={bits} tau={tau}", flush=True)
    lib = importlib.import_module("triton-kernel-test_amd._lib").load()
    L = importlib.import_module("triton-kernel-test_amd.legacy")
    l, r, x, s = _inputs(4000 + N + bits, B, M, N, K, s_rows)
    ld, rd, xd, sd = l.to(dev), r.to(dev), x.to(dev), s.to(dev)
    cap = B * M * N
    oc, q = L._encode_coo(ld, rd, xd, sd, bits, tau, cap)
    # the two-call path on the same inputs
    o2 = torch.empty((B, M, N), dtype=torch.bfloat16, device=dev)
    q2 = torch.empty_like(q)
    l2, rt, KK = L._factors(ld, rd)
    s2 = L._scale(sd, B, N)
    P = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    sp = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    assert lib.lrq_legacy_encode(P(l2), P(rt), KK, P(xd), B, M, N, xd.stride(0), xd.stride(1), P(s2), s2.shape[0],
                                 bits, float(tau), P(o2), P(q2), sp) == 0
    c2 = pkg.compact_outliers(o2, capacity=cap)
    torch.cuda.synchronize()
    n = int(oc.nnz.item())
    assert n == int(c2.nnz.item()) > 0
    assert torch.equal(q, q2)
    assert torch.equal(oc.piece_ptr, c2.piece_ptr)
    assert torch.equal(oc.indices[:, :n], c2.indices[:, :n]) and torch.equal(oc.values[:n], c2.values[:n])
    # and the reference-named wrapper returns that sparse tensor
    o_sp, q3 = pkg.low_rank_addition_fuse_compression_quantization(ld, rd, xd, sd, quantize_bit=bits, outlier=tau)
    assert torch.equal(q3, q) and torch.equal(o_sp.to_dense(), o2.view(o_sp.shape))


def _planted(seed, B, M, N, K, counts, big=20.0):
    """Legacy inputs whose outliers at tau = 8 are exactly planted entries: x = l @ r + small noise
    (|residual| < 1), then +-big at a chosen number of random columns of each 64-column piece,
    that number drawn from `counts`.  Returns l, r, x, s and the per-piece counts."""
    g = torch.Generator().manual_seed(seed)
    l = (torch.randn(M, K, generator=g) * 0.5).to(torch.bfloat16)
    r = (torch.randn(K, N, generator=g) * 0.5).to(torch.bfloat16)
    x = (l.float() @ r.float()).expand(B, M, N).clone() + 0.25 * torch.rand(B, M, N, generator=g)
    npc = N // 64
    pick = torch.randint(0, len(counts), (B, M, npc), generator=g)
    n = torch.tensor(counts)[pick]
    for idx in range(B * M * npc):
        b, rest = divmod(idx, M * npc)
        m, c = divmod(rest, npc)
        k = int(n[b, m, c])
        if k:
            cols = 64 * c + torch.randperm(64, generator=g)[:k]
            sign = torch.where(torch.rand(k, generator=g) < 0.5, -1.0, 1.0)
            x[b, m, cols] = sign * (big + torch.rand(k, generator=g))
    s = (0.05 + 0.35 * torch.rand(1, N, generator=g)).to(torch.bfloat16)
    return l, r, x.to(torch.bfloat16), s, n


# per-piece entry counts drawn from: many (a wave's entries exceed its LDS area of 512: written
# where formed) or few (gathered in LDS, written coalesced); both mix pieces a record holds (0 .. 2)
# with pieces read from their dense values
_DENSE_COUNTS = (0, 0, 1, 1, 2, 2, 3, 4, 9, 64)
_SPARSE_COUNTS = (0, 0, 0, 0, 0, 0, 1, 1, 2, 3)


@pytest.mark.parametrize("B,M,N,bits,counts", [(2, 37, 1024, 1, _DENSE_COUNTS), (2, 70, 1024, 2, _DENSE_COUNTS),
                                               (1, 100, 512, 4, _DENSE_COUNTS), (3, 20, 1024, 8, _DENSE_COUNTS),
                                               (2, 37, 1024, 1, _SPARSE_COUNTS), (2, 70, 1024, 2, _SPARSE_COUNTS),
                                               (1, 100, 512, 4, _SPARSE_COUNTS), (3, 20, 1024, 8, _SPARSE_COUNTS)])
def test_legacy_encode_coo_staged_records(pkg, dev, B, M, N, bits, counts):
    """The encode's staged records: pieces of 0, 1 and 2 entries (held by the record, entries in
    any of the piece's four 16-column lane groups) and of more (read back from their dense values),
    mixed across the waves, give the two-call path's COO exactly; and with fewer slots than entries
    the first `cap` entries and the full count."""
    print(f"[staged encode_coo] B={B} M={M} N={N} bits={bits} counts={counts}", flush=True)
    lib = importlib.import_module("triton-kernel-test_amd._lib").load()
    L = importlib.import_module("triton-kernel-test_amd.legacy")
    l, r, x, s, n = _planted(7000 + N + bits + len(set(counts)), B, M, N, 16, counts)
    tau = 8.0
    # the planted counts are the outliers the oracle finds, and every kind of piece occurs
    o_ref, _ = O.legacy_encode(bits16(l), bits16(r), bits16(x), bits16(s), bits, tau)
    per_piece = ((o_ref.reshape(B, M, N // 64, 64) & 0x7FFF) != 0).sum(-1)
    assert np.array_equal(per_piece, n.numpy())
    for k in set(counts):
        assert (per_piece == k).any(), k
    # (a wave's 256 consecutive pieces: over 512 entries for the dense draw, at most 512 for the sparse)
    waves = n.flatten()[: (n.numel() // 256) * 256].reshape(-1, 256).sum(-1)
    assert (waves > 512).all() if counts == _DENSE_COUNTS else (waves <= 512).all()
    ld, rd, xd, sd = l.to(dev), r.to(dev), x.to(dev), s.to(dev)
    total = int(n.sum())
    oc, q = L._encode_coo(ld, rd, xd, sd, bits, tau, total)
    o2 = torch.empty((B, M, N), dtype=torch.bfloat16, device=dev)
    q2 = torch.empty_like(q)
    l2, rt, KK = L._factors(ld, rd)
    s2 = L._scale(sd, B, N)
    P = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    sp = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    assert lib.lrq_legacy_encode(P(l2), P(rt), KK, P(xd), B, M, N, xd.stride(0), xd.stride(1), P(s2), s2.shape[0],
                                 bits, tau, P(o2), P(q2), sp) == 0
    c2 = pkg.compact_outliers(o2, capacity=total)
    small, _ = L._encode_coo(ld, rd, xd, sd, bits, tau, total // 3)
    torch.cuda.synchronize()
    assert np.array_equal(bits16(o2.cpu()), o_ref)
    assert int(oc.nnz.item()) == int(c2.nnz.item()) == total
    assert torch.equal(q, q2)
    assert torch.equal(oc.piece_ptr, c2.piece_ptr)
    assert torch.equal(oc.indices, c2.indices) and torch.equal(oc.values, c2.values)
    k = total // 3
    assert int(small.nnz.item()) == total
    assert torch.equal(small.piece_ptr, c2.piece_ptr)
    assert torch.equal(small.indices[:, :k], c2.indices[:, :k]) and torch.equal(small.values[:k], c2.values[:k])


# the reference decode test's outliers (low_rank_kernel_decode_speed_test.py:38-40): o = N(0,1) *
# (o > 1), about 16 % of the elements, above the density at which the decode gathers each wave's
# COO pieces into an LDS tile; random codes, per-batch scales; every bit width, ragged rows
@pytest.mark.parametrize("B,M,N,bits", [(2, 100, 1024, 2), (1, 70, 2048, 1), (2, 33, 512, 4), (1, 50, 512, 8),
                                        (4, 64, 1024, 2)])
def test_legacy_decode_dense_coo(pkg, dev, B, M, N, bits):
    print(f"[dense coo decode] B={B} M={M} N={N} bits={bits}", flush=True)
    g = torch.Generator().manual_seed(3000 + N + bits)
    l = torch.randn(M, 16, generator=g).to(torch.bfloat16)
    r = torch.randn(16, N, generator=g).to(torch.bfloat16)
    s = (torch.randn(B, N, generator=g) + 2).to(torch.bfloat16)
    q = torch.randint(0, 256, (B, M, N * bits // 8), generator=g, dtype=torch.uint8)
    o = torch.randn(B, M, N, generator=g).to(torch.bfloat16)
    o = o * (o > 1)
    ld, rd, sd, qd, od = l.to(dev), r.to(dev), s.to(dev), q.to(dev), o.to(dev)
    oc = pkg.compact_outliers(od, capacity=o.numel())
    a = pkg.low_rank_addition_fuse_decompression_dequantization(ld, rd, qd, oc, sd, quantize_bit=bits)
    b = pkg.low_rank_addition_fuse_decompression_dequantization(ld, rd, qd, od.to_sparse(), sd, quantize_bit=bits)
    c = pkg.low_rank_addition_fuse_decompression_dequantization(ld, rd, qd, od, sd, quantize_bit=bits)
    torch.cuda.synchronize()
    nnz = int(oc.nnz.item())
    assert nnz * 16 > o.numel(), "the case must take the dense-COO path"
    assert torch.equal(a, c) and torch.equal(b, c)
    xh_ref = O.legacy_decode(bits16(l), bits16(r), q.numpy(), bits16(o), bits16(s), bits)
    assert _frac_mismatch(bits16(a), xh_ref) <= TIE_BUDGET


# shapes large enough for the row-tile decode (k_legacy_rows: at least two ring rounds of 4 blocks
# per workgroup at about two workgroups per CU): 2, 4 and 8 bits, K 16 and 32, ragged rows, a last
# workgroup of 2 units (18 units per plane), the reference decode test's outliers
@pytest.mark.parametrize("B,M,N,K,bits", [(4, 4096, 4096, 16, 2), (4, 4100, 4608, 16, 2), (1, 16384, 4096, 32, 4),
                                          (2, 8192, 2048, 16, 8)])
def test_legacy_decode_row_tiles(pkg, dev, B, M, N, K, bits):
    """The row-tile decode, from COO outliers and without outliers, gives the bits of the decode
    that reads dense outliers (k_legacy_mfma), and a row sample matches the oracle."""
    print(f"[row-tile decode] B={B} M={M} N={N} K={K} bits={bits}", flush=True)
    g = torch.Generator(device=dev)
    g.manual_seed(5000 + N + bits)
    l = torch.randn(M, K, generator=g, device=dev).to(torch.bfloat16)
    r = torch.randn(K, N, generator=g, device=dev).to(torch.bfloat16)
    s = (torch.randn(B, N, generator=g, device=dev) + 2).to(torch.bfloat16)
    q = torch.randint(0, 256, (B, M, N * bits // 8), generator=g, device=dev, dtype=torch.uint8)
    o = torch.randn(B, M, N, generator=g, device=dev).to(torch.bfloat16)
    o = o * (o > 1)
    oc = pkg.compact_outliers(o, capacity=o.numel())
    dec = pkg.low_rank_addition_fuse_decompression_dequantization
    a = dec(l, r, q, oc, s, quantize_bit=bits)
    c = dec(l, r, q, o, s, quantize_bit=bits)
    a0 = dec(l, r, q, None, s, quantize_bit=bits)
    c0 = dec(l, r, q, torch.zeros_like(o), s, quantize_bit=bits)
    torch.cuda.synchronize()
    assert torch.equal(a, c), "COO row-tile decode differs from the dense-outlier decode"
    assert torch.equal(a0, c0), "outlier-free row-tile decode differs from the decode of zero outliers"
    rows = torch.tensor([0, 1, 15, 16, M // 2 + 3, M - 1])
    for bb in range(B):
        xh_ref = O.legacy_decode(bits16(l[rows]), bits16(r), q[bb][rows].cpu().numpy()[None],
                                 bits16(o[bb][rows])[None], bits16(s[bb:bb + 1]), bits)
        assert _frac_mismatch(bits16(a[bb][rows])[None], xh_ref) <= TIE_BUDGET


@pytest.mark.parametrize("M,N,K", [(256, 1024, 16), (50, 100, 20), (128, 2048, 32)])
def test_outlier_threshold_is_kthvalue(pkg, dev, M, N, K):
    """outlier_threshold = torch.kthvalue(|x[0] - l @ r|, int(numel * 0.99)) of
    low_rank_system_profile_forward.py:45, on the oracle's residual; and the extreme ranks."""
    print(f"[kth] M={M} N={N} K={K}", flush=True)
    l, r, x, _ = _inputs(3000 + N, 2, M, N, K, 1)
    xr = O.legacy_residual(bits16(l), bits16(r), bits16(x)[0])
    ld, rd, xd = l.to(dev), r.to(dev), x.to(dev)
    got = pkg.outlier_threshold(ld, rd, xd)
    want = O.kth_smallest_abs(xr, int(M * N * 0.99))
    assert got.item() == want, (got.item(), want)
    for k in (1, M * N // 3, M * N):
        assert pkg.residual_kthvalue(ld, rd, xd[0], k).item() == O.kth_smallest_abs(xr, k), k


def test_legacy_encode_coo_many_chunks(pkg, dev):
    """More than 4096 chunks of 4096 pieces (x [2, 135000, 4096], 17.3 M pieces): the staged
    scatter takes its chunk offsets from the separate chunk scan instead of summing the totals
    itself; the COO, count and piece pointers equal the two-call path's (generated on the GPU)."""
    B, M, N, K, bits, tau = 2, 135000, 4096, 16, 2, 3.5
    print(f"[staged encode_coo, many chunks] B={B} M={M} N={N}", flush=True)
    assert B * M * (N // 64) > 4096 * 4096
    lib = importlib.import_module("triton-kernel-test_amd._lib").load()
    L = importlib.import_module("triton-kernel-test_amd.legacy")
    g = torch.Generator(device=dev).manual_seed(91)
    ld = (torch.randn(M, K, generator=g, device=dev) * 0.5).to(torch.bfloat16)
    rd = (torch.randn(K, N, generator=g, device=dev) * 0.5).to(torch.bfloat16)
    xd = torch.randn(B, M, N, generator=g, device=dev).to(torch.bfloat16)
    sd = (0.05 + 0.35 * torch.rand(1, N, generator=g, device=dev)).to(torch.bfloat16)
    cap = B * M * N // 32
    oc, q = L._encode_coo(ld, rd, xd, sd, bits, tau, cap)
    o2 = torch.empty((B, M, N), dtype=torch.bfloat16, device=dev)
    q2 = torch.empty_like(q)
    l2, rt, KK = L._factors(ld, rd)
    s2 = L._scale(sd, B, N)
    P = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    sp = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    assert lib.lrq_legacy_encode(P(l2), P(rt), KK, P(xd), B, M, N, xd.stride(0), xd.stride(1), P(s2), s2.shape[0],
                                 bits, tau, P(o2), P(q2), sp) == 0
    c2 = pkg.compact_outliers(o2, capacity=cap)
    torch.cuda.synchronize()
    n = int(oc.nnz.item())
    assert n == int(c2.nnz.item()) and 0 < n <= cap
    assert torch.equal(q, q2)
    assert torch.equal(oc.piece_ptr, c2.piece_ptr)
    assert torch.equal(oc.indices[:, :n], c2.indices[:, :n]) and torch.equal(oc.values[:n], c2.values[:n])
