"""numpy restatement of the compressed-activation path (TEST INFRASTRUCTURE ONLY).

Representation conventions (all functions):
  * bf16 tensors are ``np.uint16`` arrays holding the raw bf16 bit patterns;
  * fp16 tensors are ``np.float16`` arrays;
  * packed codes are ``np.uint8`` arrays, row-planar (see ``pack_rowplanar``).

Two families are restated:

1. The reference's own PyTorch forms ("legacy mode"): low-rank subtraction with
   caller-supplied factors ``l @ r``, threshold outliers, a per-column symmetric
   scale and row-planar packing, evaluated with bf16 rounding after every torch
   op exactly as torch eager does on bf16 tensors.
     - encode  : low_rank_extraction_fuse_compression_quantization.py:153-171
     - decode  : low_rank_extraction_fuse_decompression_dequantization.py:155-165
     - naive   : low_rank_kernel_accuracy_test.py:6-16
     - add     : low_rank_extraction_speed.py:106-107
2. The compressed format the build adds (north-star "group mode"): in-kernel
   projection ``L = bf16(Y @ V)``, residual ``R = Y - L @ V^T``, asymmetric
   per-group min/max quantisation with fp16 scale/zero, optional outlier
   channels (fp16 side columns) and an optional 128-point Walsh-Hadamard
   rotation.  No reference function exists for these; they are pinned by the
   closed forms and invariants in tests/test_oracle.py.

Rounding points are explicit.  Where the GPU sums in an order the oracle cannot
reproduce (MFMA accumulation), the oracle uses the correctly rounded exact sum
(float64 accumulation, one rounding to fp32); parity tests then budget the rare
rounding-tie flips this can cause.
"""

from __future__ import annotations

import math

import numpy as np

__all__ = [
    # rounding helpers
    "bf16_round", "bf16_to_f32", "f32_to_bf16_f32", "f16_sat",
    # packing
    "pack_rowplanar", "unpack_rowplanar",
    # Walsh-Hadamard
    "sylvester", "WHT_SCALE", "wht128_chunks", "wht128_rows", "wht128_bf16",
    # group mode
    "projection", "lowrank_product", "fma32", "rcp32", "quant_groups", "dequant_groups",
    "encode", "decode", "reconstruct_f32",
    # outlier channels
    "colmax_abs", "topk_channels",
    # consumers
    "silu_bwd", "gelu_bwd", "softmax_bwd", "mul", "gemm", "gemm_t", "round_out",
    # legacy (reference torch forms)
    "legacy_matmul_bf16", "legacy_encode", "legacy_decode", "naive_roundtrip", "legacy_residual",
    "kth_smallest_abs", "to_coo",
    "lowrank_add",
]

# ---------------------------------------------------------------------------
# rounding helpers
# ---------------------------------------------------------------------------


def bf16_round(x) -> np.ndarray:
    """float32 (or float64, first rounded to float32) -> bf16 bits, round-to-nearest-even.

    NaN maps to the canonical quiet NaN 0x7FC0.  Overflow rounds to +-inf as IEEE RNE does.
    """
    x = np.asarray(x)
    if x.dtype != np.float32:
        x = x.astype(np.float32)
    b = x.view(np.uint32)
    rnd = ((b >> np.uint32(16)) & np.uint32(1)) + np.uint32(0x7FFF)
    out = ((b + rnd) >> np.uint32(16)).astype(np.uint16)
    nan = np.isnan(x)
    if nan.any():
        out = np.where(nan, np.uint16(0x7FC0), out)
    return out


def bf16_to_f32(u) -> np.ndarray:
    """bf16 bits -> float32 (exact)."""
    u = np.asarray(u, dtype=np.uint16)
    return (u.astype(np.uint32) << np.uint32(16)).view(np.float32)


def f32_to_bf16_f32(x) -> np.ndarray:
    """Round to bf16 and return the value as float32."""
    return bf16_to_f32(bf16_round(x))


def f16_sat(x) -> np.ndarray:
    """float32 -> fp16 with round-to-nearest-even, saturating at +-65504 instead of inf."""
    x = np.asarray(x, dtype=np.float32)
    return np.clip(x, np.float32(-65504.0), np.float32(65504.0)).astype(np.float16)


# ---------------------------------------------------------------------------
# row-planar packing (reference torch form)
# ---------------------------------------------------------------------------


def pack_rowplanar(codes: np.ndarray, bits: int) -> np.ndarray:
    """Pack unsigned ``bits``-wide codes along the last axis, row-planar.

    Byte ``j`` of a row holds the code of column ``j + i * (N / epp)`` in bits
    ``[bits*i, bits*i + bits)``, ``epp = 8 / bits``.
    Restates low_rank_extraction_fuse_compression_quantization.py:161-169 (with the
    accumulator zero-initialised; the reference ORs into uninitialised memory).
    """
    assert bits in (1, 2, 4, 8)
    epp = 8 // bits
    n = codes.shape[-1]
    assert n % epp == 0
    w = n // epp
    c = codes.astype(np.uint32)
    out = np.zeros(codes.shape[:-1] + (w,), dtype=np.uint32)
    for i in range(epp):
        out |= (c[..., i * w:(i + 1) * w] & np.uint32((1 << bits) - 1)) << np.uint32(bits * i)
    return out.astype(np.uint8)


def unpack_rowplanar(q: np.ndarray, bits: int) -> np.ndarray:
    """Inverse of ``pack_rowplanar``; returns unsigned codes (uint8).

    Restates low_rank_extraction_fuse_decompression_dequantization.py:157-163.
    """
    epp = 8 // bits
    w = q.shape[-1]
    qq = q.astype(np.uint32)
    out = np.empty(q.shape[:-1] + (w * epp,), dtype=np.uint8)
    mask = np.uint32((1 << bits) - 1)
    for i in range(epp):
        out[..., i * w:(i + 1) * w] = (qq >> np.uint32(bits * i)) & mask
    return out


# ---------------------------------------------------------------------------
# 128-point Walsh-Hadamard rotation (no reference function; textbook Sylvester)
# ---------------------------------------------------------------------------

WHT_SCALE = np.float32(1.0 / math.sqrt(128.0))


def sylvester(n: int) -> np.ndarray:
    """Sylvester Hadamard matrix H_n (entries +-1), H_{2n} = [[H, H], [H, -H]]."""
    h = np.ones((1, 1), dtype=np.int64)
    while h.shape[0] < n:
        h = np.block([[h, h], [h, -h]])
    assert h.shape[0] == n
    return h


_H128 = None


def wht128_chunks():
    """Column order of the rotation's accumulation: step c (0..3) adds the 32 columns
    32g + 8c + e (g < 4, e < 8) of the block, one rounding to fp32 per step."""
    return [np.array([32 * g + 8 * c + e for g in range(4) for e in range(8)]) for c in range(4)]


def wht128_rows(y: np.ndarray) -> np.ndarray:
    """Blockwise normalised WHT along the last axis (config 4; no reference function).
    Per 128-column block b and output column o:

      acc = 0;  for c in 0..3:  acc = fp32(acc + sum_{k in chunk c} H[o, k] * y[128b + k])
      out[128b + o] = fp32(acc * fp32(1/sqrt(128)))

    (chunks from ``wht128_chunks``; each step's sum is exact, as one MFMA forms it).  The
    normalised H is symmetric and its own inverse, so the function undoes itself up to
    rounding.  Pinned by: H H = 128 I, WHT(e_k) = column k / sqrt(128), norm preservation,
    agreement with the exact matrix product to fp32 rounding (tests/test_oracle.py).
    """
    global _H128
    if _H128 is None:
        _H128 = sylvester(128).astype(np.float64)
    y = np.asarray(y)
    lead, n = y.shape[:-1], y.shape[-1]
    assert n % 128 == 0, "hidden size must be a multiple of 128 for the rotation"
    yb = y.astype(np.float64).reshape(-1, n // 128, 128)
    acc = np.zeros(yb.shape, dtype=np.float32)
    for cols in wht128_chunks():
        part = yb[..., cols] @ _H128[cols, :]  # H symmetric: row-vector times H == H times column
        acc = (acc.astype(np.float64) + part).astype(np.float32)
    return (acc * WHT_SCALE).astype(np.float32).reshape(lead + (n,))


def wht128_bf16(x_bits: np.ndarray) -> np.ndarray:
    """The rotation as the kernels apply it to a bf16 tensor: bf16(wht128_rows(x))."""
    return bf16_round(wht128_rows(bf16_to_f32(x_bits)))


# ---------------------------------------------------------------------------
# group mode: projection, low-rank product, per-group quantiser
# ---------------------------------------------------------------------------


def projection(y: np.ndarray, v_bits: np.ndarray):
    """``L32 = fp32(exact(y @ V))``, ``L = bf16(L32)``.  y: float32 [M, N]; V bf16 bits [N, r].

    Returns (L bf16 bits [M, r], L32 float32).  Pinned by: orthonormal-V identities
    (projection of a vector in span(V) recovers its coefficients) and torch.matmul.
    """
    v = bf16_to_f32(v_bits).astype(np.float64)
    l32 = (y.astype(np.float64) @ v).astype(np.float32)
    return bf16_round(l32), l32


def lowrank_product(l_bits: np.ndarray, v_bits: np.ndarray, row_index=None) -> np.ndarray:
    """``L @ V^T`` with bf16 L [M', r] and V [N, r], exact in float64 (products of bf16 are
    exact; the r-term sums are exact for ordinary exponent ranges).  float64 [M, N].

    ``row_index`` optionally maps output rows to rows of L (legacy batched form).
    """
    l = bf16_to_f32(l_bits).astype(np.float64)
    if row_index is not None:
        l = l[row_index]
    v = bf16_to_f32(v_bits).astype(np.float64)
    return l @ v.T


def fma32(a, b, c) -> np.ndarray:
    """Correctly rounded float32 fused multiply-add ``round32(a*b + c)``.

    a*b is exact in float64; the float64 sum is corrected with the exact TwoSum error, so
    the one case where rounding the float64 sum to float32 could differ from rounding the
    exact value (the sum landing exactly on a float32 midpoint) is resolved by the error's sign.
    """
    a = np.asarray(a, dtype=np.float32).astype(np.float64)
    b = np.asarray(b, dtype=np.float32).astype(np.float64)
    c = np.asarray(c, dtype=np.float32).astype(np.float64)
    p = a * b
    s = p + c
    bp = s - c
    e = (p - (s - bp)) + (c - bp)          # s + e == p + c exactly
    r = s.astype(np.float32)
    d = s - r.astype(np.float64)
    away = np.nextafter(r, np.where(d >= 0, np.float32(np.inf), np.float32(-np.inf))).astype(np.float32)
    half = np.abs(away.astype(np.float64) - r.astype(np.float64)) * 0.5
    tie = (d != 0) & (np.abs(d) == half) & (e != 0)
    flip = tie & (np.sign(e) == np.sign(d))
    return np.where(flip, away, r).astype(np.float32)


def rcp32(x) -> np.ndarray:
    """Correctly rounded float32 reciprocal (what the kernels' rcp + Newton step returns for
    every positive finite fp16 input)."""
    return (np.float32(1.0) / np.asarray(x, dtype=np.float32)).astype(np.float32)


def quant_groups(r: np.ndarray, bits: int, group: int):
    """Asymmetric per-group min/max quantiser along the last axis (no reference function).

    For each group of ``group`` consecutive columns of a row:
      mn, mx   = min, max of R (fp32)
      scale_h  = fp16_rne(min((mx - mn) * fp32(1/qmax), 65504)), replaced by 1 when 0
      zero_h   = fp16_rne(clamp(mn, +-65504))
      inv      = 1 / fp32(scale_h)              (fp32, correctly rounded)
      a        = fp32(inv * fp32(1/qmax))
      b        = fp32(-fp32(zero_h) * a)
      u        = clamp(fma(R, a, b), 0, 1)      (one rounding; NaN -> 0)
      code     = rint(u * qmax)                 (exact product, round half to even),
    qmax = 2^bits - 1.  The kernels evaluate u with one clamped fma and the rounding as
    fma(u, qmax, 1.5 * 2^23), whose low mantissa bits are the code.
    Returns (codes uint8 [.., N], scale fp16 [.., N/G], zero fp16 [.., N/G],
    t = u * qmax float64 [.., N], the value that was rounded).
    Pinned by: codes in range, min/max map to the end codes, constant groups decode
    exactly, |decode - R| <= scale/2 (tests/test_oracle.py).
    """
    r = np.asarray(r, dtype=np.float32)
    lead, n = r.shape[:-1], r.shape[-1]
    assert n % group == 0
    qmax = (1 << bits) - 1
    rg = r.reshape(lead + (n // group, group))
    mn = rg.min(axis=-1)
    mx = rg.max(axis=-1)
    scale_f = (mx - mn) * np.float32(1.0 / qmax)
    scale_f = np.minimum(scale_f, np.float32(65504.0))
    scale_h = scale_f.astype(np.float16)
    scale_h = np.where(scale_h == 0, np.float16(1.0), scale_h)
    zero_h = f16_sat(mn)
    inv = rcp32(scale_h.astype(np.float32))
    a = (inv * np.float32(1.0 / qmax)).astype(np.float32)
    b = (-zero_h.astype(np.float32) * a).astype(np.float32)
    u = fma32(rg, a[..., None], b[..., None])
    u = np.where(np.isnan(u), np.float32(0.0), np.clip(u, np.float32(0.0), np.float32(1.0)))
    t = u.astype(np.float64) * qmax
    codes = np.rint(t).astype(np.uint8)
    return (codes.reshape(lead + (n,)), scale_h, zero_h, t.reshape(lead + (n,)))


def dequant_groups(codes: np.ndarray, scale_h: np.ndarray, zero_h: np.ndarray, group: int) -> np.ndarray:
    """``d = fp32(code) * fp32(scale) + fp32(zero)`` (the product is exact; one rounding)."""
    lead, n = codes.shape[:-1], codes.shape[-1]
    cg = codes.reshape(lead + (n // group, group)).astype(np.float32)
    d = cg * scale_h.astype(np.float32)[..., None] + zero_h.astype(np.float32)[..., None]
    return d.reshape(lead + (n,)).astype(np.float32)


def encode(x_bits: np.ndarray, v_bits, bits: int = 4, group: int = 64, hadamard: bool = False,
           outlier_idx=None, l_override=None) -> dict:
    """Group-mode encode of a bf16 activation x [M, N] (no reference function; north-star format).

    Steps (all on the CPU, float32 unless stated):
      side[:, k] = fp16(x[:, idx[k]])                            (outlier channels, if any)
      Y  = bf16(wht128_rows(x with the idx columns zeroed)) if hadamard, else fp32(x) with
           Y[:, idx] = 0   (the rotated activation is bf16; the channels leave before the
                            rotation, which would otherwise spread them over their blocks)
      L  = bf16(fp32(exact(Y @ V)))                              (if rank > 0)
      R  = fp32(exact(Y - L @ V^T))   (one rounding: the kernels form it as an MFMA whose
                                       accumulator input is Y, the same form the decode
                                       uses for Y'; else R = Y)
      R[:, idx] = 0   (not rotated: the rotated columns are all quantised)
      codes, scale, zero = quant_groups(R)
      packed = pack_rowplanar(codes)
    Returns a dict with the format (L, codes, scale, zero, side, idx) and the
    intermediates (Y, P, R, t, codes_unpacked) used by the tie-aware comparators.
    ``l_override`` (bf16 bits [M, r]) replaces the projection result, so the quantiser can be
    checked conditionally on a device-computed L.
    """
    x_bits = np.asarray(x_bits, dtype=np.uint16)
    m, n = x_bits.shape
    x = bf16_to_f32(x_bits)
    idx = None
    side = None
    if outlier_idx is not None and len(outlier_idx) > 0:
        idx = np.asarray(outlier_idx, dtype=np.int32)
        side = x[:, idx].astype(np.float16)
    if hadamard:
        xm = x_bits.copy()
        if idx is not None:
            xm[:, idx] = 0
        y = bf16_to_f32(wht128_bf16(xm))
    else:
        y = x.copy()
        if idx is not None:
            y[:, idx] = 0.0
    rank = 0 if v_bits is None else int(np.asarray(v_bits).shape[1])
    if rank > 0:
        if l_override is None:
            l_bits, l32 = projection(y, v_bits)
        else:
            l_bits, l32 = np.asarray(l_override, dtype=np.uint16), None
        p = lowrank_product(l_bits, v_bits)
        r = (y.astype(np.float64) - p).astype(np.float32)  # one rounding
    else:
        l_bits, l32, p = None, None, None
        r = y
    if idx is not None and not hadamard:
        r[:, idx] = 0.0
    codes, scale, zero, t = quant_groups(r, bits, group)
    return dict(L=l_bits, codes=pack_rowplanar(codes, bits), scale=scale, zero=zero, side=side,
                idx=idx, Y=y, P=p, R=r, t=t, codes_unpacked=codes, L32=l32)


def reconstruct_f32(l_bits, v_bits, packed, scale, zero, bits: int, group: int, hadamard=False,
                    side=None, idx=None) -> np.ndarray:
    """fp32 reconstruction before the final bf16 rounding (see ``decode``).  The low-rank
    term is added inside the accumulation (one rounding): ``accumulator += tl.dot(a, b)`` in
    low_rank_extraction_fuse_decompression_dequantization.py:107 is an MMA with the
    dequantised values as its accumulator input."""
    codes = unpack_rowplanar(np.asarray(packed, dtype=np.uint8), bits)
    y = dequant_groups(codes, scale, zero, group)
    if l_bits is not None and v_bits is not None and np.asarray(v_bits).shape[1] > 0:
        y = (y.astype(np.float64) + lowrank_product(l_bits, v_bits)).astype(np.float32)  # one rounding
    has_side = idx is not None and len(idx) > 0
    if hadamard:
        # rotate back, then the side columns (they were taken out before the rotation)
        y = wht128_rows(bf16_to_f32(bf16_round(y)))
    if has_side:
        y[:, np.asarray(idx)] = np.asarray(side, dtype=np.float16).astype(np.float32)
    return y


def decode(l_bits, v_bits, packed, scale, zero, bits: int, group: int, hadamard=False,
           side=None, idx=None) -> np.ndarray:
    """Group-mode decode: ``x_hat = bf16(reconstruct_f32(...))`` where

      d  = fp32(code) * scale + zero
      Y' = fp32(exact(d + L @ V^T))   (one rounding; rank > 0)
      Y'[:, idx] = side     (outlier channels; the plain format)
      X' = wht128_rows(bf16(Y')), then X'[:, idx] = side   (the rotated format: the rotation is
           its own inverse, takes bf16 input, and the side columns enter after it)
    Returns bf16 bits [M, N].
    """
    return bf16_round(reconstruct_f32(l_bits, v_bits, packed, scale, zero, bits, group, hadamard,
                                      side, idx))


# ---------------------------------------------------------------------------
# outlier channels (config 3): column abs-max + top-k
# ---------------------------------------------------------------------------


def colmax_abs(x_bits: np.ndarray) -> np.ndarray:
    """Column abs-max over all rows, float32 [N].  (No reference function; the reference's
    channel split at extraction_outlier_channel.py:11-14 takes caller indices.)"""
    return np.abs(bf16_to_f32(x_bits)).max(axis=0).astype(np.float32)


def topk_channels(colmax: np.ndarray, k: int) -> np.ndarray:
    """Indices of the ``k`` largest column abs-max values, returned sorted ascending.

    Ties are broken toward the lower column index.  Pinned by torch.topk on
    well-separated values (tests/test_oracle.py)."""
    colmax = np.asarray(colmax, dtype=np.float32)
    order = np.lexsort((np.arange(colmax.size), -colmax.astype(np.float64)))
    return np.sort(order[:k]).astype(np.int32)


# ---------------------------------------------------------------------------
# consumers: formulas evaluated in float64 on the bf16 decompressed activation,
# rounded once to bf16 by ``round_out``
# ---------------------------------------------------------------------------


def silu_bwd(x: np.ndarray, dy: np.ndarray) -> np.ndarray:
    """``dy * sigmoid(x) * (1 + x * (1 - sigmoid(x)))`` — silu_backward.py:6-8,
    extraction_fuse_silu_backward.py:10-13."""
    x = np.asarray(x, dtype=np.float64)
    s = 1.0 / (1.0 + np.exp(-x))
    return np.asarray(dy, dtype=np.float64) * (s * (1.0 + x * (1.0 - s)))


GELU_GAMMA = 0.7978845608028654
GELU_KAPPA = 0.044715


def gelu_bwd(x: np.ndarray, dy: np.ndarray) -> np.ndarray:
    """tanh-approximate GELU backward — gelu_backward.py:14-21."""
    x = np.asarray(x, dtype=np.float64)
    t = np.tanh(GELU_GAMMA * (x + GELU_KAPPA * x ** 3))
    return 0.5 * ((1.0 + t) + x * ((1.0 - t * t) * GELU_GAMMA * (1.0 + 3.0 * GELU_KAPPA * x * x))) \
        * np.asarray(dy, dtype=np.float64)


def softmax_bwd(p: np.ndarray, dp: np.ndarray) -> np.ndarray:
    """``(dp - rowsum(dp * p)) * p`` — softmax_backward.py:6-7 (row = last axis)."""
    p = np.asarray(p, dtype=np.float64)
    dp = np.asarray(dp, dtype=np.float64)
    return (dp - (dp * p).sum(axis=-1, keepdims=True)) * p


def mul(x: np.ndarray, y: np.ndarray) -> np.ndarray:
    """Elementwise product — extraction_fuse_hadamard.py:5-6 ("hadamard" there is x * y)."""
    return np.asarray(x, dtype=np.float64) * np.asarray(y, dtype=np.float64)


def gemm(x: np.ndarray, a: np.ndarray) -> np.ndarray:
    """``x @ a`` in float64 — extraction_fuse_matmul.py:5-6."""
    return np.asarray(x, dtype=np.float64) @ np.asarray(a, dtype=np.float64)


def gemm_t(x: np.ndarray, g: np.ndarray) -> np.ndarray:
    """``x^T @ g`` in float64: the LoRA factor gradient ``x.mT @ (dy @ b.mT)`` with
    g = dy @ b.mT (low_rank_system_profile_forward.py:14-18), a reduction over the rows."""
    return np.asarray(x, dtype=np.float64).T @ np.asarray(g, dtype=np.float64)


def round_out(v: np.ndarray) -> np.ndarray:
    """Round a float64 consumer result once: float64 -> float32 -> bf16 bits."""
    return bf16_round(np.asarray(v, dtype=np.float64).astype(np.float32))


# ---------------------------------------------------------------------------
# legacy mode: the reference's torch forms, bf16 rounding after each op
# ---------------------------------------------------------------------------


def legacy_matmul_bf16(l_bits: np.ndarray, r_bits: np.ndarray) -> np.ndarray:
    """``l @ r`` on bf16 tensors: fp32 accumulation (here exact, then rounded to fp32),
    result rounded to bf16.  Returns bf16 bits [M, N]."""
    prod = bf16_to_f32(l_bits).astype(np.float64) @ bf16_to_f32(r_bits).astype(np.float64)
    return bf16_round(prod.astype(np.float32))


def _bf16_op(a_f32, b_f32, op):
    return bf16_round(op(a_f32.astype(np.float32), b_f32.astype(np.float32)).astype(np.float32))


def legacy_encode(l_bits, r_bits, x_bits, s_bits, bits: int = 8, outlier: float = 5.0):
    """torch_low_rank_addition_fuse_compression_quantization
    (low_rank_extraction_fuse_compression_quantization.py:153-171), bf16 semantics:

      lr = bf16(l @ r);  xr = bf16(x - lr)
      o  = xr where |xr| > bf16(outlier) else 0;  x2 = xr - o
      c  = clamp(rint(bf16(x2 / s)), -2^(b-1), 2^(b-1)-1) + 2^(b-1)       (s broadcast per batch)
      q  = pack_rowplanar(c)
    x [B, M, N], l [M, K], r [K, N], s [B or 1, N] — all bf16 bits.
    Returns (o bf16 bits dense [B, M, N], q uint8 [B, M, N*b/8]).
    """
    x_bits = np.asarray(x_bits, dtype=np.uint16)
    lr = bf16_to_f32(legacy_matmul_bf16(l_bits, r_bits))
    x = bf16_to_f32(x_bits)
    xr = bf16_to_f32(_bf16_op(x, lr[None], np.subtract))
    tau = bf16_to_f32(bf16_round(np.float32(outlier)))
    mask = np.abs(xr) > tau
    o = np.where(mask, xr, np.float32(0.0)).astype(np.float32)
    x2 = np.where(mask, np.float32(0.0), xr).astype(np.float32)
    s = bf16_to_f32(np.asarray(s_bits, dtype=np.uint16))[:, None, :]
    d = bf16_to_f32(_bf16_op(x2, np.broadcast_to(s, x2.shape), np.divide))
    half = 1 << (bits - 1)
    c = (np.clip(np.rint(d), -half, half - 1) + half).astype(np.uint8)
    return bf16_round(o), pack_rowplanar(c, bits)


def legacy_residual(l_bits, r_bits, x_bits) -> np.ndarray:
    """``x - l @ r`` on bf16 tensors (bf16(l @ r), then the bf16 subtraction), as the encode's
    first line (low_rank_extraction_fuse_compression_quantization.py:154) and the threshold
    calibration (low_rank_system_profile_forward.py:45) compute it.  Returns bf16 bits."""
    lr = bf16_to_f32(legacy_matmul_bf16(l_bits, r_bits))
    return _bf16_op(bf16_to_f32(np.asarray(x_bits, dtype=np.uint16)), lr, np.subtract)


def kth_smallest_abs(x_bits, k: int) -> np.float32:
    """``torch.kthvalue(x.flatten().abs().to(torch.float32), k).values`` for bf16 x: the k-th
    smallest magnitude, 1-based (low_rank_system_profile_forward.py:45).
    Pinned by: torch.kthvalue on the same magnitudes (tests/test_oracle.py)."""
    a = np.abs(bf16_to_f32(np.asarray(x_bits, dtype=np.uint16)).ravel())
    return np.float32(np.partition(a, k - 1)[k - 1])


def to_coo(o_bits):
    """``o.to_sparse()`` of a bf16 tensor (low_rank_extraction_fuse_compression_quantization.py:149,
    :170): the entries whose value is not zero (bits other than +0 / -0), in row-major order;
    returns (indices int64 [ndim, nnz], value bits uint16 [nnz]).
    Pinned by: torch's to_sparse on the same tensor (tests/test_oracle.py)."""
    o_bits = np.asarray(o_bits, dtype=np.uint16)
    nz = (o_bits & 0x7FFF) != 0
    idx = np.stack(np.nonzero(nz)).astype(np.int64) if o_bits.ndim else np.zeros((0, 0), np.int64)
    return idx, o_bits[nz]


def legacy_decode(l_bits, r_bits, q, o_bits, s_bits, bits: int = 8):
    """torch_low_rank_addition_fuse_decompression_dequantization
    (low_rank_extraction_fuse_decompression_dequantization.py:155-165), bf16 semantics:

      x_hat = bf16( bf16( bf16((c - 2^(b-1)) * s) + o ) + bf16(l @ r) )
    ``o_bits`` may be None (no outliers: the add of zero is exact).  Returns bf16 bits.
    """
    c = unpack_rowplanar(np.asarray(q, dtype=np.uint8), bits).astype(np.float32) - np.float32(1 << (bits - 1))
    s = bf16_to_f32(np.asarray(s_bits, dtype=np.uint16))[:, None, :]
    a = bf16_to_f32(_bf16_op(c, np.broadcast_to(s, c.shape), np.multiply))
    if o_bits is not None:
        a = bf16_to_f32(_bf16_op(a, bf16_to_f32(o_bits), np.add))
    lr = bf16_to_f32(legacy_matmul_bf16(l_bits, r_bits))
    return _bf16_op(a, np.broadcast_to(lr[None], a.shape), np.add)


def naive_roundtrip(l_bits, r_bits, x_bits, s_bits, bits: int = 8, outlier: float = 5.0):
    """naive_quantization_dequantization (low_rank_kernel_accuracy_test.py:6-16): the
    unpacked round trip ``clamp(round(R/s)) * s + o + l @ r`` in bf16 semantics."""
    lr = bf16_to_f32(legacy_matmul_bf16(l_bits, r_bits))
    x = bf16_to_f32(np.asarray(x_bits, dtype=np.uint16))
    xr = bf16_to_f32(_bf16_op(x, lr[None], np.subtract))
    tau = bf16_to_f32(bf16_round(np.float32(outlier)))
    mask = np.abs(xr) > tau
    o = np.where(mask, xr, np.float32(0.0)).astype(np.float32)
    x2 = np.where(mask, np.float32(0.0), xr).astype(np.float32)
    s = bf16_to_f32(np.asarray(s_bits, dtype=np.uint16))[:, None, :]
    d = bf16_to_f32(_bf16_op(x2, np.broadcast_to(s, x2.shape), np.divide))
    half = 1 << (bits - 1)
    qv = np.clip(np.rint(d), -half, half - 1).astype(np.float32)
    a = bf16_to_f32(_bf16_op(qv, np.broadcast_to(s, qv.shape), np.multiply))
    a = bf16_to_f32(_bf16_op(a, o, np.add))
    return _bf16_op(a, np.broadcast_to(lr[None], a.shape), np.add)


def lowrank_add(l_bits, r_bits, x_bits):
    """torch_low_rank_addition (low_rank_extraction_speed.py:106-107): ``bf16(x + bf16(l @ r))``."""
    lr = bf16_to_f32(legacy_matmul_bf16(l_bits, r_bits))
    x = bf16_to_f32(np.asarray(x_bits, dtype=np.uint16))
    return _bf16_op(x, np.broadcast_to(lr, x.shape) if x.ndim == 2 else np.broadcast_to(lr[None], x.shape),
                    np.add)
