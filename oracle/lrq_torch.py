"""PyTorch-eager fp32 restatement of the path on the CPU (TEST INFRASTRUCTURE ONLY).

This is the CPU baseline ``bench.py`` times (``cpu_baseline``, kind "port"): the same
algorithms as ``lrq_oracle`` written as vectorised torch ops on CPU tensors, so they use every
host core through torch's intra-op threads.  It is never the product and never imported by
the ``triton-kernel-test_amd`` package.

Numerics: fp32 matmuls (torch's blocked summation order), bf16 / fp16 rounding at the same
points as ``lrq_oracle``.  Where ``lrq_oracle`` sums exactly in float64 this module sums in
fp32, so a value sitting on a rounding boundary can land one code / one ulp away;
``tests/test_oracle.py`` pins this module against ``lrq_oracle`` (codes equal except for such
flips, decode within one bf16 ulp) at sizes the numpy oracle finishes quickly.

Reference formulas restated (file:line in Ther-nullptr/Triton-Kernel-Test):
  * legacy encode / decode: low_rank_extraction_fuse_compression_quantization.py:153-171,
    low_rank_extraction_fuse_decompression_dequantization.py:155-165 (bf16 torch ops as written)
  * SiLU / GELU / softmax backward: silu_backward.py:6-8, gelu_backward.py:14-21,
    softmax_backward.py:6-7
  * LoRA factor gradients: low_rank_system_profile_forward.py:14-18
The group-mode format (projection, per-group asymmetric quantiser, rotation, outlier channels)
has no reference function; it follows ``lrq_oracle.encode`` / ``decode`` step by step.
"""

from __future__ import annotations

import math

import torch

__all__ = ["pack_rowplanar", "unpack_rowplanar", "wht128", "encode", "decode", "silu_bwd", "gelu_bwd",
           "softmax_bwd", "legacy_encode", "legacy_decode", "to_coo"]

_H = {}


def _h128(device) -> torch.Tensor:
    """Normalised Sylvester H_128 (fp32): H_{2n} = [[H, H], [H, -H]], scaled by 1/sqrt(128)."""
    if device not in _H:
        h = torch.ones((1, 1))
        while h.shape[0] < 128:
            h = torch.cat([torch.cat([h, h], 1), torch.cat([h, -h], 1)], 0)
        _H[device] = (h * (1.0 / math.sqrt(128.0))).to(device)
    return _H[device]


def wht128(y: torch.Tensor) -> torch.Tensor:
    """Blockwise normalised WHT-128 along the last axis, fp32 (``lrq_oracle.wht128_rows``)."""
    n = y.shape[-1]
    return (y.reshape(-1, 128) @ _h128(y.device)).reshape(y.shape[:-1] + (n,))


def pack_rowplanar(codes: torch.Tensor, bits: int) -> torch.Tensor:
    """Row-planar packing (``lrq_oracle.pack_rowplanar``): byte j of a row holds column
    j + p*N/NP in bits [p*bits, (p+1)*bits)."""
    np_ = 8 // bits
    m, n = codes.shape
    planes = codes.to(torch.int32).reshape(m, np_, n // np_)
    out = planes[:, 0].clone()
    for p in range(1, np_):
        out |= planes[:, p] << (p * bits)
    return out.to(torch.uint8)


def unpack_rowplanar(q: torch.Tensor, bits: int) -> torch.Tensor:
    np_ = 8 // bits
    mask = (1 << bits) - 1
    qi = q.to(torch.int32)
    return torch.cat([(qi >> (p * bits)) & mask for p in range(np_)], dim=-1).to(torch.uint8)


def encode(x: torch.Tensor, V: torch.Tensor | None, bits: int = 4, group: int = 64, hadamard: bool = False,
           outlier_idx: torch.Tensor | None = None) -> dict:
    """Group-mode encode of a bf16 x [M, N] on the CPU (``lrq_oracle.encode``, fp32 sums)."""
    m, n = x.shape
    y = x.float()
    side = None
    if outlier_idx is not None and outlier_idx.numel() > 0:
        side = x[:, outlier_idx.long()].half()
        y[:, outlier_idx.long()] = 0.0  # before the rotation
    if hadamard:
        y = wht128(y).bfloat16().float()
    L = None
    if V is not None:
        v = V.float()
        L = (y @ v).bfloat16()
        r = y - L.float() @ v.T
    else:
        r = y
    if side is not None and not hadamard:
        r[:, outlier_idx.long()] = 0.0
    qmax = (1 << bits) - 1
    rg = r.reshape(m, n // group, group)
    mn, mx = rg.amin(-1), rg.amax(-1)
    scale = ((mx - mn) * (1.0 / qmax)).clamp(max=65504.0).half()
    scale = torch.where(scale == 0, torch.ones_like(scale), scale)
    zero = mn.clamp(-65504.0, 65504.0).half()
    a = (1.0 / scale.float()) * (1.0 / qmax)
    b = -zero.float() * a
    u = torch.addcmul(b[..., None], rg, a[..., None]).clamp_(0.0, 1.0)
    codes = torch.round(u * qmax).to(torch.uint8).reshape(m, n)
    return dict(L=L, codes=pack_rowplanar(codes, bits), scale=scale, zero=zero, side=side, idx=outlier_idx)


def decode(e: dict, V: torch.Tensor | None, bits: int, group: int, hadamard: bool = False) -> torch.Tensor:
    """Group-mode decode (``lrq_oracle.decode``): bf16(codes*scale + zero + L V^T), side
    columns substituted (the rotated format: the rotation undone on the bf16 result first)."""
    codes = unpack_rowplanar(e["codes"], bits)
    m, n = codes.shape
    y = (codes.float().reshape(m, n // group, group) * e["scale"].float()[..., None]
         + e["zero"].float()[..., None]).reshape(m, n)
    if V is not None and e["L"] is not None:
        y = torch.addmm(y, e["L"].float(), V.float().T)
    side = e.get("side")
    if side is not None and not hadamard:
        y[:, e["idx"].long()] = side.float()
    if hadamard:
        y = wht128(y.bfloat16().float())
        if side is not None:
            y[:, e["idx"].long()] = side.float()  # after the rotation
    return y.bfloat16()


def silu_bwd(x: torch.Tensor, dy: torch.Tensor) -> torch.Tensor:
    """dy * s(x) (1 + x (1 - s(x))) in fp32, rounded once (silu_backward.py:6-8)."""
    xf = x.float()
    s = torch.sigmoid(xf)
    return (dy.float() * s * (1.0 + xf * (1.0 - s))).bfloat16()


def gelu_bwd(x: torch.Tensor, dy: torch.Tensor) -> torch.Tensor:
    """tanh-approximate GELU backward in fp32 (gelu_backward.py:14-21)."""
    xf = x.float()
    g, k = 0.7978845608028654, 0.044715
    t = torch.tanh(g * (xf + k * xf ** 3))
    return (0.5 * ((1.0 + t) + xf * ((1.0 - t * t) * g * (1.0 + 3.0 * k * xf * xf))) * dy.float()).bfloat16()


def softmax_bwd(p: torch.Tensor, dp: torch.Tensor) -> torch.Tensor:
    """(dp - rowsum(dp p)) p in fp32 (softmax_backward.py:6-7)."""
    pf, dpf = p.float(), dp.float()
    return ((dpf - (dpf * pf).sum(-1, keepdim=True)) * pf).bfloat16()


def legacy_encode(l: torch.Tensor, r: torch.Tensor, x: torch.Tensor, s: torch.Tensor, bits: int, outlier: float):
    """The reference's torch encode on bf16 CPU tensors
    (low_rank_extraction_fuse_compression_quantization.py:153-171, without its `.cuda()`):
    returns (dense outliers bf16, codes uint8 row-planar)."""
    xr = x - l @ r
    o = xr * (xr.abs() > outlier)
    x2 = xr - o
    half = 1 << (bits - 1)
    c = (torch.clamp(torch.round(x2 / s.unsqueeze(-2)), -half, half - 1).to(torch.int16) + half).to(torch.uint8)
    return o, pack_rowplanar(c.reshape(-1, c.shape[-1]), bits).reshape(c.shape[:-1] + (-1,))


def legacy_decode(l: torch.Tensor, r: torch.Tensor, q: torch.Tensor, o: torch.Tensor | None, s: torch.Tensor,
                  bits: int) -> torch.Tensor:
    """The reference's torch decode (low_rank_extraction_fuse_decompression_dequantization.py:155-165)."""
    c = unpack_rowplanar(q.reshape(-1, q.shape[-1]), bits).reshape(q.shape[:-1] + (-1,))
    a = (c.to(torch.int16) - (1 << (bits - 1))).to(torch.int8) * s.unsqueeze(-2)
    if o is not None:
        a = a + o
    return a + l @ r


def to_coo(o: torch.Tensor):
    """The reference's `o.to_sparse()` (…compression_quantization.py:149)."""
    return o.to_sparse()
