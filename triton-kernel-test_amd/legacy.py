"""The reference's own operator names and signatures ("legacy mode"), on liblrq.so.

Same positional signatures, argument meanings and assertion messages as the reference's
Python wrappers; the arithmetic follows the reference's torch forms (bf16 rounding after
every op, row-planar packing, per-batch scale rows) rather than its Triton kernels, whose
defects (s[0] only, tile-planar packing, unmasked scratch stores) are not reproduced.

  low_rank_addition_fuse_compression_quantization      low_rank_extraction_fuse_compression_quantization.py:118
  low_rank_addition_fuse_decompression_dequantization  low_rank_extraction_fuse_decompression_dequantization.py:116
  low_rank_addition                                    low_rank_extraction_speed.py:77
  triton_silu_backward_fuse_extraction                 extraction_fuse_silu_backward.py:192
  triton_silu_backward_add_extraction                  extraction_fuse_silu_backward.py:324 (returns the result)
  triton_hadamard_fuse_extraction                      extraction_fuse_hadamard.py:185
  triton_hadamard_add_extraction                       extraction_fuse_hadamard.py:317 (returns the result)
  triton_matmul_decompress                             extraction_fuse_matmul.py:224
  triton_silu_backward                                 silu_backward.py:54
  triton_gelu_backward                                 gelu_backward.py:73
  triton_softmax_backward                              softmax_backward.py:45
  triton_hadamard                                      extraction_fuse_hadamard.py:62
  torch_extract_unstructured                           extraction_outlier_channel.py:5
  torch_extract_channel                                extraction_outlier_channel.py:11

The outliers these functions return sparse (``o.to_sparse()`` in the reference) are compacted on
the GPU by ``lrq_coo_compact``; ``compact_outliers`` / ``legacy_encode_coo`` keep them as a
``LegacyOutliers`` (COO buffers with the entry count on the device, no host synchronisation),
which the decode reads directly.  ``outlier_threshold`` is the reference's calibration
``torch.kthvalue(|x[0] - L_x @ R_x|, k)`` (low_rank_system_profile_forward.py:45) on the GPU.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import Optional

import torch

from . import _lib
from ._lib import call
from .api import _p, _require_device, _stream

__all__ = [
    "low_rank_addition_fuse_compression_quantization",
    "low_rank_addition_fuse_decompression_dequantization",
    "low_rank_addition",
    "triton_silu_backward_fuse_extraction",
    "triton_silu_backward_add_extraction",
    "triton_hadamard_fuse_extraction",
    "triton_hadamard_add_extraction",
    "triton_matmul_decompress",
    "triton_silu_backward",
    "triton_gelu_backward",
    "triton_softmax_backward",
    "triton_hadamard",
    "torch_extract_unstructured",
    "torch_extract_channel",
    "LegacyOutliers",
    "compact_outliers",
    "legacy_encode_coo",
    "outlier_threshold",
    "residual_kthvalue",
]

_OP_STORE, _OP_SILU, _OP_MUL = 0, 1, 2


def _factors(l: torch.Tensor, r: torch.Tensor):
    """Zero-pad the rank to 16 or 32 (as the reference pads K < 16 to 16,
    low_rank_extraction_fuse_compression_quantization.py:126-129) and build rt = r^T [N, K]."""
    _require_device(l, r)
    M, K = l.shape
    K2, N = r.shape
    if K2 != K:
        raise AssertionError("Incompatible dimensions")
    if K > 32:
        raise ValueError("liblrq supports low-rank factors of rank <= 32")
    kp = 16 if K <= 16 else 32
    if kp != K:
        l = torch.cat([l, torch.zeros((M, kp - K), device=l.device, dtype=l.dtype)], dim=1)
        r = torch.cat([r, torch.zeros((kp - K, N), device=r.device, dtype=r.dtype)], dim=0)
    l = l.to(torch.bfloat16).contiguous()
    r = r.to(torch.bfloat16).contiguous()
    rt = torch.empty((N, kp), dtype=torch.bfloat16, device=r.device)
    call("lrq_transpose_bf16", _p(r), kp, N, _p(rt), _stream(r.device))
    return l, rt, kp


def _scale(s: torch.Tensor, B: int, N: int) -> torch.Tensor:
    _require_device(s)
    if s.dim() == 1:
        s = s.unsqueeze(0)
    if s.shape[-1] != N or s.shape[0] not in (1, B):
        raise ValueError(f"s must be [B or 1, N] = [{B} or 1, {N}], got {tuple(s.shape)}")
    return s.to(torch.bfloat16).contiguous()


def _bits(quantize_bit: int) -> int:
    if quantize_bit not in (1, 2, 4, 8):
        raise ValueError("quantize_bit must be 1, 2, 4 or 8")
    return int(quantize_bit)


@dataclass
class LegacyOutliers:
    """Legacy-format outliers as COO on the device: ``indices`` int64 [3, cap] (b, m, n; entry e
    in column e), ``values`` bf16 [cap], ``nnz`` int64 [1] (device; may exceed cap, then the
    entries past cap were not written), ``piece_ptr`` int64 [B*M*ceil(N/64) + 1] (first entry of
    each 64-column piece of a row), ``shape`` the dense shape (1 to 3 dims)."""
    indices: torch.Tensor
    values: torch.Tensor
    nnz: torch.Tensor
    piece_ptr: torch.Tensor
    shape: tuple

    @property
    def capacity(self) -> int:
        return self.values.numel()

    def check(self) -> "LegacyOutliers":
        """Raise if the compaction dropped entries (nnz > capacity); one host synchronisation."""
        n = int(self.nnz.item())
        if n > self.capacity:
            raise RuntimeError(f"{n} outliers exceed the capacity {self.capacity}; compact again with a larger one")
        return self

    def to_sparse(self) -> torch.Tensor:
        """The coalesced sparse COO tensor (one host synchronisation, for the entry count)."""
        n = int(self.check().nnz.item())
        nd = len(self.shape)
        return torch.sparse_coo_tensor(self.indices[3 - nd:, :n], self.values[:n], self.shape, is_coalesced=True,
                                       check_invariants=True)


def _bmn(shape) -> tuple:
    if len(shape) == 3:
        return tuple(shape)
    if len(shape) == 2:
        return (1, shape[0], shape[1])
    if len(shape) == 1:
        return (1, 1, shape[0])
    raise ValueError("outlier tensors have 1 to 3 dimensions")


def _coo_buffers(B: int, M: int, N: int, cap: int, dev):
    npc = (N + 63) // 64
    wsb = _lib.call_raw("lrq_coo_workspace", B, M, N)
    _lib.check(min(wsb, 0), "lrq_coo_workspace")
    return dict(idx=torch.empty((3, cap), dtype=torch.int64, device=dev),
                vals=torch.empty((cap,), dtype=torch.bfloat16, device=dev),
                nnz=torch.empty((1,), dtype=torch.int64, device=dev),
                ptr=torch.empty((B * M * npc + 1,), dtype=torch.int64, device=dev),
                ws=torch.empty((max(wsb, 8) + 7) // 8, dtype=torch.int64, device=dev))


def compact_outliers(o: torch.Tensor, capacity: Optional[int] = None) -> LegacyOutliers:
    """Dense bf16 outliers -> LegacyOutliers on the GPU (lrq_coo_compact), no synchronisation.
    capacity defaults to max(1024, numel / 32)."""
    _require_device(o)
    o = o.to(torch.bfloat16).contiguous()
    B, M, N = _bmn(tuple(o.shape))
    cap = max(1024, o.numel() // 32) if capacity is None else int(capacity)
    dev = o.device
    bf = _coo_buffers(B, M, N, cap, dev)
    with torch.cuda.device(dev):
        call("lrq_coo_compact", _p(o), B, M, N, _p(bf["idx"]), cap, _p(bf["vals"]), cap, _p(bf["nnz"]),
             _p(bf["ptr"]), _p(bf["ws"]), bf["ws"].numel() * 8, _stream(dev))
    return LegacyOutliers(bf["idx"], bf["vals"], bf["nnz"], bf["ptr"], tuple(o.shape))


def _to_sparse(o: torch.Tensor) -> torch.Tensor:
    """``o.to_sparse()`` through the GPU compaction (one synchronisation, as to_sparse has).
    Tensors of more than 3 dimensions are compacted as [prod(leading), M, N] and their leading
    index unravelled afterwards (row-major order is the same)."""
    shape = tuple(o.shape)
    o3 = o.reshape((-1,) + shape[-2:]) if len(shape) > 3 else o
    c = compact_outliers(o3)
    n = int(c.nnz.item())
    if n > c.capacity:
        c = compact_outliers(o3, capacity=n)
    sp = c.to_sparse()
    if len(shape) <= 3:
        return sp
    lead, rest = sp.indices()[0], []
    for d in reversed(shape[:-2]):
        rest.append(lead % d)
        lead = torch.div(lead, d, rounding_mode="floor")
    ind = torch.cat([torch.stack(rest[::-1]), sp.indices()[1:]])
    return torch.sparse_coo_tensor(ind, sp.values(), shape, is_coalesced=True)


def _coo_pieces(o, B: int, M: int, N: int):
    """(piece_ptr, cols, vals, entries) of the decode for LegacyOutliers or a sparse COO tensor."""
    if isinstance(o, LegacyOutliers):
        return o.piece_ptr, o.indices[2], o.values, o.capacity
    o = o.coalesce()
    ind = o.indices()
    b, m, n = ([torch.zeros_like(ind[0])] * (3 - ind.shape[0])) + list(ind)
    npc = (N + 63) // 64
    pid = (b * M + m) * npc + torch.div(n, 64, rounding_mode="floor")
    ptr = torch.searchsorted(pid, torch.arange(B * M * npc + 1, device=pid.device, dtype=torch.int64))
    return ptr, n.contiguous(), o.values().to(torch.bfloat16).contiguous(), int(n.numel())


def _encode_coo(l, r, x, s, bits: int, outlier: float, capacity: Optional[int]):
    """lrq_legacy_encode_coo: (LegacyOutliers, q).  Its dense outlier buffer is working memory
    (only pieces with more entries than the encode's staged records hold are written to it)."""
    _require_device(x)
    M, _ = l.shape
    _, N = r.shape
    B = x.shape[0]
    if tuple(x.shape) != (B, M, N):
        raise ValueError(f"x must be [B, {M}, {N}]")
    if x.stride(2) != 1:
        x = x.contiguous()
    with torch.cuda.device(x.device):
        l2, rt, K = _factors(l, r)
        s2 = _scale(s, B, N)
        o = torch.empty((B, M, N), device=x.device, dtype=torch.bfloat16)
        q = torch.empty((B, M, N // (8 // bits)), device=x.device, dtype=torch.uint8)
        cap = max(1024, o.numel() // 32) if capacity is None else int(capacity)
        bf = _coo_buffers(B, M, N, cap, x.device)
        # the encode stages each piece's count and first entries as it quantises (the
        # compaction's first pass)
        call("lrq_legacy_encode_coo", _p(l2), _p(rt), K, _p(x), B, M, N, x.stride(0), x.stride(1), _p(s2),
             s2.shape[0], bits, float(outlier), _p(o), _p(q), _p(bf["idx"]), cap, _p(bf["vals"]), cap,
             _p(bf["nnz"]), _p(bf["ptr"]), _p(bf["ws"]), bf["ws"].numel() * 8, _stream(x.device))
    return LegacyOutliers(bf["idx"], bf["vals"], bf["nnz"], bf["ptr"], tuple(o.shape)), q


def low_rank_addition_fuse_compression_quantization(l, r, x, s, quantize_bit=8, outlier=5.):
    """Encode x[B, M, N] - l@r: threshold outliers (returned sparse COO, like the reference) and
    symmetric per-column quantisation with row-planar packing.  Returns (o, q)."""
    assert l.shape[1] == r.shape[0], "Incompatible dimensions"
    assert l.is_contiguous(), "Matrix A must be contiguous"
    assert r.is_contiguous(), "Matrix B must be contiguous"
    bits = _bits(quantize_bit)
    oc, q = _encode_coo(l, r, x, s, bits, outlier, None)
    n = int(oc.nnz.item())  # the host synchronisation to_sparse has too
    if n > oc.capacity:  # more entries than the default buffers hold: again, with room for all
        oc, q = _encode_coo(l, r, x, s, bits, outlier, n)
    return oc.to_sparse(), q


def legacy_encode_coo(l, r, x, s, quantize_bit=8, outlier=5., capacity: Optional[int] = None):
    """low_rank_addition_fuse_compression_quantization with the outliers kept as LegacyOutliers
    (compacted on the GPU, the encode doing the compaction's count pass, entry count left on the
    device): no host synchronisation.  A decode of it reads at most `capacity` entries;
    ``LegacyOutliers.check()`` tells whether any were dropped."""
    return _encode_coo(l, r, x, s, _bits(quantize_bit), outlier, capacity)


def low_rank_addition_fuse_decompression_dequantization(l, r, q, o, s, quantize_bit=8, outlier=5.):
    """Decode: bf16(bf16(bf16(c*s) + o) + bf16(l@r)).  ``o`` may be sparse COO, LegacyOutliers,
    dense or None; COO outliers are read by the decode kernel itself (no dense tensor)."""
    assert l.shape[1] == r.shape[0], "Incompatible dimensions"
    assert l.is_contiguous(), "Matrix A must be contiguous"
    assert r.is_contiguous(), "Matrix B must be contiguous"
    bits = _bits(quantize_bit)
    _require_device(q)
    M, _ = l.shape
    _, N = r.shape
    B = q.shape[0]
    q = q.contiguous()
    coo = isinstance(o, LegacyOutliers) or (o is not None and o.is_sparse)
    if o is not None and not isinstance(o, LegacyOutliers):
        _require_device(o)
        if not coo:
            o = o.to(torch.bfloat16).contiguous()
    with torch.cuda.device(q.device):
        l2, rt, K = _factors(l, r)
        s2 = _scale(s, B, N)
        x = torch.empty((B, M, N), device=q.device, dtype=torch.bfloat16)
        if coo:
            ptr, cols, vals, n = _coo_pieces(o, B, M, N)
            call("lrq_legacy_decode_coo", _p(l2), _p(rt), K, _p(q), _p(ptr), _p(cols), _p(vals), n, _p(s2),
                 s2.shape[0], B, M, N, bits, _p(x), _stream(q.device))
        else:
            call("lrq_legacy_decode", _p(l2), _p(rt), K, _p(q), _p(o), _p(s2), s2.shape[0], B, M, N, bits,
                 _p(x), _stream(q.device))
    return x


def residual_kthvalue(l, r, x, k: int) -> torch.Tensor:
    """torch.kthvalue(|x - l @ r|.flatten().to(torch.float32), k).values for x[M, N] (bf16
    arithmetic of the reference: the residual rounded to bf16), on the GPU: a 0-dim fp32 device
    tensor (lrq_legacy_kth_residual)."""
    _require_device(x)
    M, _ = l.shape
    _, N = r.shape
    if x.dim() != 2 or tuple(x.shape) != (M, N):
        raise ValueError(f"x must be [{M}, {N}]")
    x = x.to(torch.bfloat16)
    if x.stride(1) != 1:
        x = x.contiguous()
    out = torch.empty((), dtype=torch.float32, device=x.device)
    ws = torch.empty((256,), dtype=torch.int64, device=x.device)
    with torch.cuda.device(x.device):
        l2, rt, K = _factors(l, r)
        call("lrq_legacy_kth_residual", _p(l2), _p(rt), K, _p(x), M, N, x.stride(0), int(k), _p(out), _p(ws),
             ws.numel() * 8, _stream(x.device))
    return out


def outlier_threshold(l, r, x, fraction: float = 0.01) -> torch.Tensor:
    """The reference's threshold calibration (low_rank_system_profile_forward.py:45):
    kthvalue of |x[0] - l @ r| at k = int(x[0].numel() * (1 - fraction)), on the GPU (a 0-dim
    fp32 device tensor; the reference takes ``.item()`` of it)."""
    x0 = x[0] if x.dim() == 3 else x
    return residual_kthvalue(l, r, x0, int(x0.numel() * (1 - fraction)))


def low_rank_addition(l, r, x):
    """x + l @ r with the torch form's bf16 rounding (low_rank_extraction_speed.py:106-107)."""
    assert l.shape[1] == r.shape[0], "Incompatible dimensions"
    assert l.is_contiguous(), "Matrix A must be contiguous"
    assert r.is_contiguous(), "Matrix B must be contiguous"
    _require_device(x)
    M, _ = l.shape
    _, N = r.shape
    B = x.shape[0]
    x = x.contiguous()
    with torch.cuda.device(x.device):
        l2, rt, K = _factors(l, r)
        o = torch.empty((B, M, N), device=x.device, dtype=torch.bfloat16)
        call("lrq_lowrank_add", _p(l2), _p(rt), K, _p(x), B, M, N, _p(o), _stream(x.device))
    return o


def _legacy_fused(op, l, r, q, s, b, quantize_bit):
    bits = _bits(quantize_bit)
    _require_device(q)
    M, _ = l.shape
    _, N = r.shape
    B = q.shape[0]
    q = q.contiguous()
    if b is not None:
        _require_device(b)
        if tuple(b.shape) != (B, M, N):
            raise ValueError(f"second operand must be [{B}, {M}, {N}]")
        b = b.to(torch.bfloat16).contiguous()
    with torch.cuda.device(q.device):
        l2, rt, K = _factors(l, r)
        s2 = _scale(s, B, N)
        c = torch.empty((B, M, N), device=q.device, dtype=torch.bfloat16)
        call("lrq_legacy_fused", _p(l2), _p(rt), K, _p(q), _p(s2), s2.shape[0], B, M, N, bits, op, _p(b),
             _p(c), _stream(q.device))
    return c


def triton_silu_backward_fuse_extraction(l, r, q, s, b, quantize_bit=2):
    """SiLU backward of the decompressed activation, decompression fused in-kernel."""
    return _legacy_fused(_OP_SILU, l, r, q, s, b, quantize_bit)


def triton_hadamard_fuse_extraction(l, r, q, s, b, quantize_bit=2):
    """Elementwise product of the decompressed activation with b, fused in-kernel."""
    return _legacy_fused(_OP_MUL, l, r, q, s, b, quantize_bit)


def triton_silu_backward_add_extraction(l, r, q, s, b, quantize_bit=2):
    """Unfused: decode kernel, then the SiLU-backward kernel (the reference returns None here)."""
    a = _legacy_fused(_OP_STORE, l, r, q, s, None, quantize_bit)
    return triton_silu_backward(a, b)


def triton_hadamard_add_extraction(l, r, q, s, b, quantize_bit=2):
    """Unfused: decode kernel, then the elementwise-product kernel (the reference returns None)."""
    a = _legacy_fused(_OP_STORE, l, r, q, s, None, quantize_bit)
    return triton_hadamard(a, b)


def triton_matmul_decompress(q, l, r, s, y, quantize_bit=2):
    """decode(q) @ y per batch: x_hat[B, M, N] @ y[B, N, n] -> bf16 [B, M, n], in one kernel
    (lrq_legacy_dequant_gemm): x_hat is rebuilt in registers and fed to the product MFMA, never
    stored; fp32 sums rounded to bf16 once.  Output widths that are not a multiple of 16 are
    computed on y zero-padded to one."""
    bits = _bits(quantize_bit)
    _require_device(q, y)
    M, _ = l.shape
    _, N = r.shape
    B = q.shape[0]
    if y.dim() != 3 or y.shape[0] != B or y.shape[1] != N:
        raise ValueError(f"y must be [{B}, {N}, n], got {tuple(y.shape)}")
    n = y.shape[2]
    q = q.contiguous()
    y = y.to(torch.bfloat16)
    npad = (n + 15) // 16 * 16
    if npad != n:
        y = torch.nn.functional.pad(y, (0, npad - n))
    y = y.contiguous()
    with torch.cuda.device(q.device):
        l2, rt, K = _factors(l, r)
        s2 = _scale(s, B, N)
        o = torch.empty((B, M, npad), device=q.device, dtype=torch.bfloat16)
        if n > 0 and M > 0:
            call("lrq_legacy_dequant_gemm", _p(l2), _p(rt), K, _p(q), _p(s2), s2.shape[0], B, M, N, bits, _p(y), npad,
                 npad, _p(o), npad, _stream(q.device))
    return o if npad == n else o[..., :n].contiguous()


def _dense(op, x, y):
    _require_device(x, y)
    if x.shape != y.shape:
        raise AssertionError("shape mismatch")
    x = x.to(torch.bfloat16).contiguous()
    y = y.to(torch.bfloat16).contiguous()
    o = torch.empty_like(x)
    with torch.cuda.device(x.device):
        call("lrq_dense_elementwise", op, _p(x), _p(y), _p(o), x.numel(), _stream(x.device))
    return o


def triton_silu_backward(x, g):
    """g * s(x)(1 + x(1 - s(x))) in fp32, rounded once (silu_backward.py:54-69)."""
    return _dense(0, x, g)


def triton_gelu_backward(x, g):
    """tanh-GELU backward in fp32, rounded once (gelu_backward.py:73-88)."""
    return _dense(1, x, g)


def triton_hadamard(a, b):
    """a * b (extraction_fuse_hadamard.py:62-73)."""
    return _dense(2, a, b)


def triton_softmax_backward(y, grad_y):
    """(g - rowsum(g * y)) * y over the last axis (softmax_backward.py:45-61)."""
    _require_device(y, grad_y)
    assert grad_y.shape == y.shape
    n = y.shape[-1]
    y2 = y.to(torch.bfloat16).contiguous()
    g2 = grad_y.to(torch.bfloat16).contiguous()
    o = torch.empty_like(y2)
    with torch.cuda.device(y.device):
        call("lrq_dense_softmax_bwd", _p(y2), _p(g2), _p(o), y2.numel() // n, n, _stream(y.device))
    return o


def torch_extract_unstructured(x, threshold):
    """(x * (|x| > threshold)).to_sparse() and the remainder x - that, on the HIP kernel
    (the comparison is made in bf16, as for a bf16 tensor against a scalar)."""
    _require_device(x)
    x2 = x.to(torch.bfloat16).contiguous()
    o = torch.empty_like(x2)
    rest = torch.empty_like(x2)
    tau = float(threshold.item() if isinstance(threshold, torch.Tensor) else threshold)
    with torch.cuda.device(x2.device):
        call("lrq_threshold_split", _p(x2), x2.numel(), tau, _p(o), _p(rest), _stream(x2.device))
    return _to_sparse(o), rest


def torch_extract_channel(x, channel_index):
    """Returns (x[:, channel_index, :], x) after zeroing those rows of x in place — the
    reference's axis (dim 1) and in-place behaviour, kept for drop-in use.  For hidden-channel
    outliers of the compressed format see ``outlier_channels`` / ``encode(outlier_idx=...)``."""
    _require_device(x)
    if x.dim() != 3 or x.dtype != torch.bfloat16 or not x.is_contiguous():
        raise ValueError("x must be a contiguous bf16 [B, M, N] tensor")
    idx = torch.as_tensor(channel_index, device=x.device).to(torch.int32).contiguous()
    if idx.numel() != torch.unique(idx).numel():
        raise ValueError("channel_index must not repeat")
    B, M, N = x.shape
    out = torch.empty((B, idx.numel(), N), dtype=x.dtype, device=x.device)
    with torch.cuda.device(x.device):
        call("lrq_gather_rows_zero", _p(x), B, M, N, _p(idx), idx.numel(), _p(out), _stream(x.device))
    return out, x
