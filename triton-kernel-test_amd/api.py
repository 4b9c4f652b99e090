"""Python operator API over liblrq.so (group mode — the north-star compressed format).

Functions take and return torch tensors on a ROCm device and launch the HIP kernels on
torch's current stream.  There is no CPU path: host tensors raise ``ValueError`` and a
missing library raises ``RuntimeError``.

Reference call surface this mirrors (file:line in Ther-nullptr/Triton-Kernel-Test):
  encode                      <- low_rank_addition_fuse_compression_quantization
                                 (low_rank_extraction_fuse_compression_quantization.py:118)
  decode                      <- low_rank_addition_fuse_decompression_dequantization
                                 (low_rank_extraction_fuse_decompression_dequantization.py:116)
  silu_backward_compressed    <- triton_silu_backward_fuse_extraction (extraction_fuse_silu_backward.py:192)
  mul_compressed              <- triton_hadamard_fuse_extraction (extraction_fuse_hadamard.py:185)
  dequant_gemm                <- triton_matmul_decompress (extraction_fuse_matmul.py:224)
  gelu_backward_compressed    <- triton_gelu_backward formula (gelu_backward.py:14-21), fused
  softmax_backward_compressed <- triton_softmax_backward formula (softmax_backward.py:6-7), fused
  outlier_channels            <- torch_extract_channel (extraction_outlier_channel.py:11-14), with
                                 the channel set chosen by column abs-max instead of given
The reference-named legacy functions live in ``legacy.py``.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import Optional

import torch

from . import _lib
from ._lib import LrqTensors, call

__all__ = [
    "LowRankBasis", "CompressedActivation", "encode", "decode", "silu_backward_compressed",
    "gelu_backward_compressed", "mul_compressed", "softmax_backward_compressed", "dequant_gemm",
    "dequant_gemm_t", "dequant_gemm_t_noalloc", "lora_grads", "outlier_channels", "column_absmax", "topk_channels",
    "wht128",
]


def _p(t: Optional[torch.Tensor]):
    return ctypes.c_void_p(t.data_ptr() if t is not None else 0)


def _stream(device: torch.device):
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def _require_device(*ts):
    for t in ts:
        if t is not None and not t.is_cuda:
            raise ValueError("liblrq works on ROCm device tensors only (there is no CPU path); got a "
                             f"tensor on {t.device}")


def _rows_view(x: torch.Tensor) -> tuple[torch.Tensor, int, int, int]:
    """View x[..., N] as a 2-D [rows, N] operand with unit inner stride; returns (x2, rows, N, ld)."""
    if x.dim() < 1:
        raise ValueError("activation must have at least one dimension")
    n = x.shape[-1]
    if x.dim() == 2 and x.stride(1) == 1:
        return x, x.shape[0], n, x.stride(0)
    x2 = x.reshape(-1, n)
    if x2.stride(-1) != 1:
        x2 = x2.contiguous()
    return x2, x2.shape[0], n, x2.stride(0)


class LowRankBasis:
    """An orthonormal basis V[N, r] (bf16, device) used for the projection.

    ``Vt`` (the [r, N] transpose the projection operand wants) is built once on the
    device by ``lrq_transpose_bf16`` and cached, like a pre-packed weight.
    """

    def __init__(self, V: torch.Tensor):
        _require_device(V)
        if V.dtype != torch.bfloat16 or V.dim() != 2:
            raise ValueError("basis V must be a bf16 [N, r] tensor")
        self.V = V.contiguous()
        self._vt: Optional[torch.Tensor] = None

    @property
    def hidden(self) -> int:
        return self.V.shape[0]

    @property
    def rank(self) -> int:
        return self.V.shape[1]

    @property
    def Vt(self) -> torch.Tensor:
        if self._vt is None:
            vt = torch.empty((self.rank, self.hidden), dtype=torch.bfloat16, device=self.V.device)
            with torch.cuda.device(self.V.device):
                call("lrq_transpose_bf16", _p(self.V), self.hidden, self.rank, _p(vt), _stream(self.V.device))
            self._vt = vt
        return self._vt


@dataclass
class CompressedActivation:
    """The compressed form of an activation x[..., N]; see include/lrq.h for the layout."""

    codes: torch.Tensor                 # uint8 [rows, N*bits/8], row-planar
    qparams: torch.Tensor               # fp16 [rows, U, NP, 2]: per unit, (scale, zero) of each plane
    L: Optional[torch.Tensor]           # bf16 [rows, r]
    basis: Optional[LowRankBasis]
    side: Optional[torch.Tensor]        # fp16 [rows, k]
    idx: Optional[torch.Tensor]         # int32 [k] (-1: an entry dropped as invalid, see _outlier_index)
    shape: tuple
    bits: int
    group: int
    hadamard: bool = False

    @property
    def rows(self) -> int:
        return self.codes.shape[0]

    @property
    def hidden(self) -> int:
        return self.shape[-1]

    @property
    def rank(self) -> int:
        return 0 if self.basis is None else self.basis.rank

    @property
    def device(self) -> torch.device:
        return self.codes.device

    def _per_group(self, which: int) -> torch.Tensor:
        # qparams[r, u, i] belongs to group i*U + u of the row (plane i, unit u)
        q = self.qparams[..., which]                      # [rows, U, NP]
        return q.permute(0, 2, 1).reshape(self.rows, -1)  # [rows, N/group], column order

    @property
    def scale(self) -> torch.Tensor:
        """Per-group scale, fp16 [rows, N/group] in column order (a copy)."""
        return self._per_group(0)

    @property
    def zero(self) -> torch.Tensor:
        """Per-group zero point (group minimum), fp16 [rows, N/group] in column order (a copy)."""
        return self._per_group(1)

    def nbytes(self) -> int:
        n = self.codes.numel() + 2 * self.qparams.numel()
        if self.L is not None:
            n += 2 * self.L.numel()
        if self.side is not None:
            n += 2 * self.side.numel() + 4 * self.idx.numel()
        return n

    def descriptor(self, for_encode: bool = False) -> LrqTensors:
        t = LrqTensors()
        t.rows, t.hidden = self.rows, self.hidden
        t.rank, t.bits, t.group = self.rank, self.bits, self.group
        # encode sets the flag itself when it hands the library the unrotated activation (see
        # ``encode``); every other entry point sees the flag
        t.flags = _lib.LRQ_FLAG_HADAMARD if (self.hadamard and not for_encode) else 0
        if self.rank:
            t.L, t.ld_L = self.L.data_ptr(), self.L.stride(0)
            t.V = self.basis.V.data_ptr()
            if for_encode:
                t.Vt = self.basis.Vt.data_ptr()
        t.codes, t.ld_codes = self.codes.data_ptr(), self.codes.stride(0)
        t.qparams, t.ld_qp = self.qparams.data_ptr(), self.qparams.stride(0)
        if self.idx is not None and self.idx.numel() > 0:
            t.outlier_idx, t.n_outlier = self.idx.data_ptr(), self.idx.numel()
            t.side, t.ld_side = self.side.data_ptr(), self.side.stride(0)
        return t


def _alloc(rows: int, n: int, bits: int, group: int, rank: int, k: int, device) -> dict:
    # Code rows are N*bits/8 bytes: a multiple of the group (>= 64), so 16-byte aligned.
    np_ = 8 // bits
    if n % (group * np_) != 0:
        raise ValueError(f"hidden size {n} must be a multiple of group*8/bits = {group * np_}")
    return dict(
        codes=torch.empty((rows, n * bits // 8), dtype=torch.uint8, device=device),
        qparams=torch.empty((rows, n // (group * np_), np_, 2), dtype=torch.float16, device=device),
        L=torch.empty((rows, rank), dtype=torch.bfloat16, device=device) if rank else None,
        side=torch.empty((rows, k), dtype=torch.float16, device=device) if k else None,
    )


def _outlier_index(idx, n: int, device) -> tuple[torch.Tensor, bool]:
    """The outlier-channel index list as int32 on the device, and whether it was sanitized.
    Indices the host holds (a list, numpy array or CPU tensor) must be distinct and in [0, n):
    ValueError otherwise.  A device tensor (e.g. topk_channels' output) is not read back: an
    entry outside [0, n) or a repeat of an earlier entry becomes -1, which every kernel skips,
    and its side column is zero-filled (no host synchronisation)."""
    if isinstance(idx, torch.Tensor) and idx.is_cuda:
        _require_device(idx)
        idx = idx.to(torch.int32).contiguous()
        k = idx.numel()
        if k == 0:
            return idx, False
        valid = (idx >= 0) & (idx < n)
        vals, perm = torch.sort(idx, stable=True)
        first = torch.ones(k, dtype=torch.bool, device=idx.device)
        first[1:] = vals[1:] != vals[:-1]
        first_at = torch.empty_like(first)
        first_at[perm] = first
        return torch.where(valid & first_at, idx, torch.full_like(idx, -1)), True
    h = torch.as_tensor(idx).reshape(-1).to(torch.int64)
    if h.numel() and (int(h.min()) < 0 or int(h.max()) >= n):
        raise ValueError(f"outlier_idx entries must lie in [0, {n})")
    if h.numel() != torch.unique(h).numel():
        raise ValueError("outlier_idx entries must be distinct")
    return h.to(torch.int32).to(device).contiguous(), False


def encode(x: torch.Tensor, basis: Optional[LowRankBasis | torch.Tensor] = None, *, bits: int = 4,
           group_size: int = 64, hadamard: bool = False, outlier_idx: Optional[torch.Tensor] = None,
           _twopass: bool = False) -> CompressedActivation:
    """Compress a bf16 activation x[..., N].

    ``basis``: the rank-r orthonormal V[N, r] (or a ``LowRankBasis``); None for rank 0.
    ``outlier_idx``: column indices kept as fp16 side columns (see ``outlier_channels``);
    host-held indices must be distinct and in range, device-held ones are sanitized on the device
    (``_outlier_index``).
    """
    _require_device(x)
    if x.dtype != torch.bfloat16:
        raise ValueError("activation must be bf16")
    if isinstance(basis, torch.Tensor):
        basis = LowRankBasis(basis)
    x2, rows, n, ldx = _rows_view(x)
    if basis is not None and basis.hidden != n:
        raise ValueError(f"basis has {basis.hidden} rows, activation hidden size is {n}")
    rank = 0 if basis is None else basis.rank
    sanitized = False
    if outlier_idx is not None:
        outlier_idx, sanitized = _outlier_index(outlier_idx, n, x.device)
    k = 0 if outlier_idx is None else outlier_idx.numel()
    bufs = _alloc(rows, n, bits, group_size, rank, k, x.device)
    if sanitized and k:
        bufs["side"].zero_()  # the side columns of dropped indices read as zeros
    c = CompressedActivation(codes=bufs["codes"], qparams=bufs["qparams"], L=bufs["L"],
                             basis=basis, side=bufs["side"], idx=outlier_idx if k else None,
                             shape=tuple(x.shape), bits=bits, group=group_size, hadamard=hadamard)
    t = c.descriptor(for_encode=True)
    with torch.cuda.device(x.device):
        if hadamard:
            # rotated format: the library rotates x as it reads it where it can (flagged
            # descriptor); otherwise y = bf16(WHT128(x)) into a temporary, then the plain encode
            t.flags = _lib.LRQ_FLAG_HADAMARD
            st = _lib.call_raw("lrq_encode_twopass" if _twopass else "lrq_encode", ctypes.byref(t), _p(x2), ldx,
                               _stream(x.device))
            if st != _lib.LRQ_ERR_UNSUPPORTED or k:
                # (outlier channels leave X before the rotation: no rotated copy can stand in)
                _lib.check(st, "lrq_encode")
                return c
            t.flags = 0
            y = torch.empty((rows, n), dtype=torch.bfloat16, device=x.device)
            call("lrq_wht128", _p(x2), ldx, rows, n, _p(y), n, _stream(x.device))
            x2, ldx = y, n
        call("lrq_encode_twopass" if _twopass else "lrq_encode", ctypes.byref(t), _p(x2), ldx,
             _stream(x.device))
    return c


def wht128(x: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """bf16(normalised blockwise WHT-128(x)) along the last axis (its own inverse up to
    rounding).  ``out`` may be ``x`` (in place)."""
    _require_device(x)
    if x.dtype != torch.bfloat16:
        raise ValueError("wht128 takes bf16")
    x2, rows, n, ldx = _rows_view(x)
    o = torch.empty(x.shape, dtype=torch.bfloat16, device=x.device) if out is None else out
    if o.shape != x.shape or o.dtype != torch.bfloat16 or not o.is_contiguous():
        raise ValueError("out must be a contiguous bf16 tensor of x's shape")
    with torch.cuda.device(x.device):
        call("lrq_wht128", _p(x2), ldx, rows, n, _p(o), n, _stream(x.device))
    return o


def _out_like(c: CompressedActivation, out: Optional[torch.Tensor]) -> torch.Tensor:
    if out is None:
        return torch.empty(c.shape, dtype=torch.bfloat16, device=c.device)
    if out.shape != torch.Size(c.shape) or out.dtype != torch.bfloat16 or not out.is_contiguous():
        raise ValueError("out must be a contiguous bf16 tensor of the activation's shape")
    return out


def _operand(c: CompressedActivation, y: torch.Tensor, name: str) -> tuple[torch.Tensor, int]:
    _require_device(y)
    if tuple(y.shape) != tuple(c.shape) or y.dtype != torch.bfloat16:
        raise ValueError(f"{name} must be bf16 with the activation's shape {c.shape}")
    y2, _, _, ld = _rows_view(y)
    return y2, ld


def decode(c: CompressedActivation, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Reconstruct x_hat (bf16, the activation's shape)."""
    o = _out_like(c, out)
    t = c.descriptor()
    with torch.cuda.device(c.device):
        call("lrq_decode", ctypes.byref(t), _p(o), c.hidden, _stream(c.device))
    return o


def _fused(name: str, c: CompressedActivation, y: torch.Tensor, argname: str) -> torch.Tensor:
    if c.hadamard or (c.idx is not None and name == "lrq_softmax_bwd"):
        # the library's two-kernel forms of these (decode into the output, then the dense op in
        # place) take rows of exactly `hidden` elements
        y = y.contiguous()
    y2, ldy = _operand(c, y, argname)
    o = _out_like(c, None)
    t = c.descriptor()
    with torch.cuda.device(c.device):
        call(name, ctypes.byref(t), _p(y2), ldy, _p(o), c.hidden, _stream(c.device))
    return o


def silu_backward_compressed(c: CompressedActivation, grad_output: torch.Tensor) -> torch.Tensor:
    """dX = dY * s(x)(1 + x(1 - s(x))) with x = decode(c), decompressed in-kernel."""
    return _fused("lrq_silu_bwd", c, grad_output, "grad_output")


def gelu_backward_compressed(c: CompressedActivation, grad_output: torch.Tensor) -> torch.Tensor:
    """tanh-approximate GELU backward on x = decode(c), decompressed in-kernel."""
    return _fused("lrq_gelu_bwd", c, grad_output, "grad_output")


def mul_compressed(c: CompressedActivation, y: torch.Tensor) -> torch.Tensor:
    """decode(c) * y elementwise (the reference's "hadamard" consumer)."""
    return _fused("lrq_mul", c, y, "y")


def softmax_backward_compressed(c: CompressedActivation, grad_p: torch.Tensor) -> torch.Tensor:
    """dS = P (dP - rowsum(dP P)) with P = decode(c); rows are the softmax rows."""
    return _fused("lrq_softmax_bwd", c, grad_p, "grad_p")


def dequant_gemm(c: CompressedActivation, a: torch.Tensor, out_dtype=torch.float32) -> torch.Tensor:
    """decode(c) @ a with a[N, n] bf16; fp32 accumulate, output fp32 or bf16."""
    _require_device(a)
    if a.dtype != torch.bfloat16 or a.dim() != 2 or a.shape[0] != c.hidden:
        raise ValueError("a must be bf16 [N, n]")
    a = a.contiguous()
    n_out = a.shape[1]
    if out_dtype not in (torch.float32, torch.bfloat16):
        raise ValueError("out_dtype must be float32 or bfloat16")
    o = torch.empty((c.rows, n_out), dtype=out_dtype, device=c.device)
    t = c.descriptor()
    with torch.cuda.device(c.device):
        call("lrq_dequant_gemm", ctypes.byref(t), _p(a), n_out, _p(o), n_out,
             1 if out_dtype == torch.float32 else 0, _stream(c.device))
    return o.reshape(tuple(c.shape[:-1]) + (n_out,))


def dequant_gemm_t(c: CompressedActivation, g: torch.Tensor, out_dtype=torch.float32) -> torch.Tensor:
    """decode(c)^T @ g with g[rows, n] bf16 (n = 16 or 32), reduced over the rows: the LoRA
    factor gradient x^T (dy B^T) of compute_lora_gradient (low_rank_system_profile_forward.py:14-18)
    read from the codes.  fp32 accumulate; output [N, n] fp32 or bf16."""
    _require_device(g)
    g2 = g.reshape(-1, g.shape[-1]) if g.dim() >= 2 else g
    if g.dtype != torch.bfloat16 or g.dim() < 2 or g2.shape[0] != c.rows:
        raise ValueError("g must be bf16 [rows, n] (leading dimensions those of the activation)")
    if out_dtype not in (torch.float32, torch.bfloat16):
        raise ValueError("out_dtype must be float32 or bfloat16")
    g2 = g2.contiguous()
    n_out = g2.shape[1]
    t = c.descriptor()
    ws_bytes = _lib.call_raw("lrq_dequant_gemm_t_workspace", ctypes.byref(t), n_out)
    if ws_bytes < 0:
        _lib.check(ws_bytes, "lrq_dequant_gemm_t_workspace")
    ws = torch.empty((max(ws_bytes, 16) + 15) // 16 * 4, dtype=torch.float32, device=c.device)
    o = torch.empty((c.hidden, n_out), dtype=out_dtype, device=c.device)
    with torch.cuda.device(c.device):
        call("lrq_dequant_gemm_t", ctypes.byref(t), _p(g2), n_out, n_out, _p(o), n_out,
             1 if out_dtype == torch.float32 else 0, _p(ws), ws.numel() * 4, _stream(c.device))
    return o


def lora_grads(c: CompressedActivation, a: torch.Tensor, g: torch.Tensor, xa_dtype=torch.bfloat16,
               da_dtype=torch.float32) -> tuple[torch.Tensor, torch.Tensor]:
    """(decode(c) @ a, decode(c)^T @ g) — the two products of compute_lora_gradient
    (low_rank_system_profile_forward.py:14-18) that read the saved x, from one pass over the codes
    where the format allows it (int4 / g64 / rank 16, n = 16, rows of a multiple of 512 columns,
    not rotated); otherwise ``dequant_gemm`` and ``dequant_gemm_t``.  a: bf16 [N, n]; g: bf16
    [rows, n]."""
    _require_device(a, g)
    g2 = g.reshape(-1, g.shape[-1]) if g.dim() >= 2 else g
    if a.dtype != torch.bfloat16 or a.dim() != 2 or a.shape[0] != c.hidden:
        raise ValueError("a must be bf16 [N, n]")
    if g.dtype != torch.bfloat16 or g.dim() < 2 or g2.shape[0] != c.rows or g2.shape[1] != a.shape[1]:
        raise ValueError("g must be bf16 [rows, n] (leading dimensions those of the activation)")
    for d in (xa_dtype, da_dtype):
        if d not in (torch.float32, torch.bfloat16):
            raise ValueError("output dtypes must be float32 or bfloat16")
    n_out = a.shape[1]
    t = c.descriptor()
    ws_bytes = _lib.call_raw("lrq_lora_grads_workspace", ctypes.byref(t), n_out)
    if ws_bytes == _lib.LRQ_ERR_UNSUPPORTED:
        xa = dequant_gemm(c, a, out_dtype=xa_dtype).reshape(-1, n_out)
        return xa, dequant_gemm_t(c, g2, out_dtype=da_dtype)
    if ws_bytes < 0:
        _lib.check(ws_bytes, "lrq_lora_grads_workspace")
    a2, g2 = a.contiguous(), g2.contiguous()
    ws = torch.empty((max(ws_bytes, 16) + 15) // 16 * 4, dtype=torch.float32, device=c.device)
    xa = torch.empty((c.rows, n_out), dtype=xa_dtype, device=c.device)
    da = torch.empty((c.hidden, n_out), dtype=da_dtype, device=c.device)
    with torch.cuda.device(c.device):
        call("lrq_lora_grads", ctypes.byref(t), _p(a2), n_out, _p(g2), n_out, n_out, _p(xa), n_out,
             1 if xa_dtype == torch.float32 else 0, _p(da), n_out, 1 if da_dtype == torch.float32 else 0,
             _p(ws), ws.numel() * 4, _stream(c.device))
    return xa, da


def dequant_gemm_t_noalloc(c: CompressedActivation, g: torch.Tensor, out: torch.Tensor) -> torch.Tensor:
    """``dequant_gemm_t`` into a caller-provided ``out`` [N, n] (fp32 or bf16, contiguous), with
    the library's own device scratch in place of a workspace: neither this function nor the
    library allocates device memory, so it can run under HIP graph capture.  ``g`` must be a
    contiguous bf16 [rows, n].  Calls that overlap on one GPU share the scratch and race."""
    _require_device(g, out)
    if g.dtype != torch.bfloat16 or g.dim() != 2 or g.shape[0] != c.rows or not g.is_contiguous():
        raise ValueError("g must be a contiguous bf16 [rows, n]")
    n_out = g.shape[1]
    if out.dtype not in (torch.float32, torch.bfloat16) or tuple(out.shape) != (c.hidden, n_out) \
            or not out.is_contiguous():
        raise ValueError("out must be a contiguous fp32 or bf16 [N, n]")
    t = c.descriptor()
    with torch.cuda.device(c.device):
        call("lrq_dequant_gemm_t_noalloc", ctypes.byref(t), _p(g), n_out, n_out, _p(out), n_out,
             1 if out.dtype == torch.float32 else 0, _stream(c.device))
    return out


def column_absmax(x: torch.Tensor) -> torch.Tensor:
    """max over rows of |x[..., c]| as fp32 [N]."""
    _require_device(x)
    x2, rows, n, ldx = _rows_view(x)
    out = torch.empty((n,), dtype=torch.float32, device=x.device)
    with torch.cuda.device(x.device):
        call("lrq_colmax", _p(x2), ldx, rows, n, _p(out), _stream(x.device))
    return out


def topk_channels(colmax: torch.Tensor, k: int) -> torch.Tensor:
    """Indices of the k largest entries, ascending (ties toward the lower index)."""
    _require_device(colmax)
    colmax = colmax.to(torch.float32).contiguous()
    idx = torch.empty((k,), dtype=torch.int32, device=colmax.device)
    with torch.cuda.device(colmax.device):
        call("lrq_topk", _p(colmax), colmax.numel(), k, _p(idx), _stream(colmax.device))
    return idx


def outlier_channels(x: torch.Tensor, k: int) -> torch.Tensor:
    """The k hidden channels with the largest column abs-max (int32, ascending)."""
    return topk_channels(column_absmax(x), k)
