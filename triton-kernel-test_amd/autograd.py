"""Compress-on-save: the compressed format inside autograd.

The reference's system profiles run the path between a LoRA layer's forward and its
gradient: ``compute_lora`` (low_rank_system_profile_forward.py:8-12) produces y, the
activation x is compressed (``:50``), and before ``compute_lora_gradient`` (``:14-18``) it is
decompressed again (low_rank_system_profile_backward.py:55-61).  This module makes that
round trip part of autograd:

* ``compute_lora`` / ``compute_lora_gradient`` keep the reference's formulas (the weight is a
  dense [out, in] tensor here; the reference passes a Linear module to the forward).
* ``LoRALinearCompressed`` is an autograd Function whose forward is ``compute_lora`` and which
  saves x in the compressed format; its backward returns dx, dA and dB of
  ``compute_lora_gradient`` (W is frozen, as in the reference's LoRA setting).  With
  ``fused=True`` (the default) x is never decoded: dA = x^T (dy B^T) and x A come from the codes,
  in one pass for both (``lora_grads``: int4 / g64 / rank 16, LoRA rank 16) or from the
  transposed dequant-GEMM and the dequant-GEMM (LoRA rank 16 or 32, plain format); otherwise,
  or for other shapes, x is decoded and the formulas run on it.
* ``compressed_saved_tensors`` is a ``torch.autograd.graph.saved_tensors_hooks`` context that
  stores every saved bf16 activation with a suitable last dimension in the compressed format
  and decodes it when backward asks for it, for any model.
* ``fit_basis`` builds the rank-r basis V from a sample of activation rows (top right singular
  vectors), the counterpart of the reference's low-rank factors of x.

The compression is lossy: gradients are those of the decoded activations.
"""

from __future__ import annotations

from typing import Callable, Optional

import torch

from .api import CompressedActivation, LowRankBasis, decode, encode, lora_grads

__all__ = ["compute_lora", "compute_lora_gradient", "LoRALinearCompressed", "lora_linear_compressed",
           "compressed_saved_tensors", "fit_basis"]


def compute_lora(x: torch.Tensor, w: torch.Tensor, a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """y = x W^T + (x A) B (low_rank_system_profile_forward.py:8-12; W [out, in]).  Leading
    dimensions are folded into the rows, so every product is a plain 2-D GEMM."""
    x2 = _flat(x)
    y = x2 @ w.mT + (x2 @ a) @ b
    return y.reshape(x.shape[:-1] + (w.shape[0],))


def compute_lora_gradient(dy: torch.Tensor, x: torch.Tensor, w: torch.Tensor, a: torch.Tensor,
                          b: torch.Tensor):
    """(dx, dA, dB) of ``compute_lora`` (low_rank_system_profile_forward.py:14-18, with the
    weight in [out, in] layout: the reference's ``w.mT`` is W^T's transpose there)."""
    dx = dy @ (w + b.mT @ a.mT)
    da = x.mT @ (dy @ b.mT)
    db = (x @ a).mT @ dy
    return dx, da, db


def _flat(t: torch.Tensor) -> torch.Tensor:
    return t.reshape(-1, t.shape[-1])


class LoRALinearCompressed(torch.autograd.Function):
    """y = compute_lora(x, W, A, B); x is saved compressed (bits, group, optional basis).

    Gradients: dx, dA, dB of compute_lora_gradient on the decoded x; W gets none.  ``fused``
    reads the codes directly for dA and x A (no decoded x), see the module docstring."""

    @staticmethod
    def forward(ctx, x, w, a, b, basis: Optional[LowRankBasis], bits: int, group: int, fused: bool = True):
        y = compute_lora(x, w, a, b)
        ctx.c = encode(x.detach(), basis, bits=bits, group_size=group)
        ctx.fused = fused
        ctx.save_for_backward(w, a, b)
        return y

    @staticmethod
    def backward(ctx, dy):
        w, a, b = ctx.saved_tensors
        c, ctx.c = ctx.c, None
        dy2 = _flat(dy)
        if ctx.fused and _codes_gemm_ok(c, a, dy2):
            dx = dy2 @ (w + b.mT @ a.mT)
            # x A and x^T (dy B^T) from one pass over the codes where the format allows it
            xa, da = lora_grads(c, a, dy2 @ b.mT, xa_dtype=a.dtype, da_dtype=torch.float32)
            da = da.to(a.dtype)
            db = xa.mT @ dy2  # (x A)^T dy
        else:
            dx, da, db = compute_lora_gradient(dy2, _flat(decode(c)), w, a, b)
        return dx.reshape(dy.shape[:-1] + (w.shape[1],)), None, da, db, None, None, None, None


def _codes_gemm_ok(c: CompressedActivation, a: torch.Tensor, dy2: torch.Tensor) -> bool:
    """The dequant-GEMMs serve LoRA rank 16 / 32 on the plain (unrotated, no outlier
    channels) format with bf16 operands."""
    return (a.shape[1] in (16, 32) and not c.hadamard and c.idx is None and a.dtype == torch.bfloat16
            and dy2.dtype == torch.bfloat16)


def lora_linear_compressed(x, w, a, b, basis: Optional[LowRankBasis] = None, bits: int = 4, group: int = 64,
                           fused: bool = True):
    return LoRALinearCompressed.apply(x, w, a, b, basis, bits, group, fused)


class compressed_saved_tensors(torch.autograd.graph.saved_tensors_hooks):
    """Store saved activations compressed while this context is active.

    A saved tensor is compressed when it is a CUDA bf16 tensor produced by an operation (not
    a leaf: weights and inputs are saved as they are), its last dimension N is a multiple of
    group * 8 / bits, it holds at least ``min_numel`` elements, and ``accept(t)`` (if given)
    returns True.  ``basis_for(N)`` may return a LowRankBasis for that width (rank 0 when it
    returns None or is not given).  ``stats`` counts the tensors and bytes compressed.
    """

    def __init__(self, bits: int = 4, group: int = 64,
                 basis_for: Optional[Callable[[int], Optional[LowRankBasis]]] = None,
                 min_numel: int = 1 << 16, accept: Optional[Callable[[torch.Tensor], bool]] = None):
        np_ = 8 // bits
        self.stats = {"compressed": 0, "kept": 0, "bytes_in": 0, "bytes_out": 0}

        def pack(t: torch.Tensor):
            ok = (t.is_cuda and t.dtype == torch.bfloat16 and t.dim() >= 1 and t.grad_fn is not None
                  and t.shape[-1] % (group * np_) == 0 and t.numel() >= min_numel
                  and (accept is None or accept(t)))
            if not ok:
                self.stats["kept"] += 1
                return t
            basis = basis_for(t.shape[-1]) if basis_for is not None else None
            c = encode(t.detach(), basis, bits=bits, group_size=group)
            self.stats["compressed"] += 1
            self.stats["bytes_in"] += 2 * t.numel()
            self.stats["bytes_out"] += c.nbytes()
            return c

        def unpack(c):
            if isinstance(c, CompressedActivation):
                return decode(c)
            return c

        super().__init__(pack, unpack)


def fit_basis(x_sample: torch.Tensor, rank: int) -> LowRankBasis:
    """The top-``rank`` right singular vectors of a sample of rows x_sample[..., N] (fp32 SVD),
    as an orthonormal bf16 V[N, rank] on x_sample's device."""
    xs = _flat(x_sample).to(torch.float32)
    _, _, vh = torch.linalg.svd(xs, full_matrices=False)
    v = vh[:rank].mT.contiguous()
    return LowRankBasis(v.to(torch.bfloat16))
