"""Comparators for HIP-vs-oracle parity (test infrastructure).

Bars:
  * packed codes, scales, zeros, index sets: bit-exact, except rounding-tie flips, which
    must stay under 1e-4 of codes;
  * fused floating-point outputs: max-abs <= 1e-2 and relative-L2 <= 1e-3 against the
    oracle's decompress-then-op result (formula in float64 on the bf16 x_hat, rounded
    once to bf16).
"""

from __future__ import annotations

import numpy as np
import torch

import oracle as O

TIE_BUDGET = 1e-4
MAX_ABS = 1e-2
REL_L2 = 1e-3


def bits16(t: torch.Tensor) -> np.ndarray:
    """bf16/fp16 tensor -> uint16 bit patterns (numpy)."""
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def f16(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().numpy().astype(np.float16)


def from_bits(a: np.ndarray, device) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16).to(device)


def ulp_diff_bf16(a_bits: np.ndarray, b_bits: np.ndarray) -> np.ndarray:
    """|a - b| in bf16 ulps via the ordered integer mapping of the bit patterns."""
    def ordered(u):
        u = u.astype(np.int32)
        return np.where(u & 0x8000, 0x8000 - (u & 0x7FFF), u + 0x8000)
    return np.abs(ordered(a_bits) - ordered(b_bits))


def assert_decode_close(dev_bits: np.ndarray, ref_bits: np.ndarray, what: str, frac=1e-3, abs_tol=2.0 ** -20) -> dict:
    """Decoded bf16 vs the oracle's: at most one bf16 ulp apart, on at most ``frac`` of the
    elements, except where the reconstruction cancels to a tiny value.  The MFMA forms
    code*scale + zero + L V^T (terms of order one) in fp32 accumulation, which can sit a few
    2^-24-sized steps from the exact sum; at a result near zero that is several bf16 ulps, so
    there the bar is an absolute one (abs_tol, far below any quantisation step)."""
    d = ulp_diff_bf16(dev_bits, ref_bits)
    a = O.bf16_to_f32(dev_bits).astype(np.float64)
    b = O.bf16_to_f32(ref_bits).astype(np.float64)
    far = (d > 1) & (np.abs(a - b) > abs_tol)
    rep = dict(max_ulp=int(d.max()) if d.size else 0, frac_ulp=float((d > 0).mean()) if d.size else 0.0,
               n_cancel=int(((d > 1) & ~far).sum()), n_far=int(far.sum()))
    assert rep["n_far"] == 0 and rep["frac_ulp"] <= frac, f"{what}: {rep}"
    return rep


def assert_projection_close(l_bits: np.ndarray, y: np.ndarray, v_bits: np.ndarray, what: str, frac=1e-3) -> dict:
    """Device L (bf16 of fp32 sums of y V) vs the exact projection y V (float64).  The device
    rounds each 32-term MFMA step, the two accumulator chains and the partials of each wave or
    slab: at most 16 fp32 roundings on the way of any term, each below 2^-24 times the running
    sum of magnitudes S = |y| |V|.  Bar: every element within one bf16 ulp of the exact value
    plus 2^-19 S (twice that bound), and one-ulp flips against the oracle's L (the exact sum
    rounded once) on at most ``frac`` of the elements.  Where L cancels to a value much below S
    the fp32 steps are several bf16 ulps of it; a wrong partial or row is off by far more."""
    yv = np.asarray(y, dtype=np.float64)
    v = O.bf16_to_f32(v_bits).astype(np.float64)
    exact = yv @ v
    big = np.abs(yv) @ np.abs(v)
    dev = O.bf16_to_f32(l_bits).astype(np.float64)
    ulp = np.exp2(np.floor(np.log2(np.maximum(np.abs(exact), 1e-30))) - 7)
    tol = ulp + 2.0 ** -19 * big
    d = ulp_diff_bf16(l_bits, O.bf16_round(exact.astype(np.float32)))
    rep = dict(max_ulp=int(d.max()) if d.size else 0, frac_ulp=float((d > 0).mean()) if d.size else 0.0,
               worst=float((np.abs(dev - exact) / tol).max()) if d.size else 0.0)
    assert rep["worst"] <= 1.0 and rep["frac_ulp"] <= frac, f"{what}: {rep}"
    return rep


def assert_rotated_close(dev_bits: np.ndarray, ref_bits: np.ndarray, what: str, frac=1e-2, k=4) -> dict:
    """Rotated-format decode (x_hat = bf16(WHT128(y))) vs the oracle's.  A one-ulp difference in
    one reconstructed value y (the MFMA's fp32 sum at rank 32, see assert_decode_close) moves
    all 128 outputs of its block by ulp(y)/sqrt(128), which flips some of them by an ulp and,
    where an output cancels to a small value, by several.  Bar: every element within one ulp of
    its own plus k such moves at the block's largest magnitude, flips on at most ``frac``."""
    a = O.bf16_to_f32(dev_bits).astype(np.float64)
    b = O.bf16_to_f32(ref_bits).astype(np.float64)
    rows, n = b.shape
    blk = np.abs(b).reshape(rows, n // 128, 128).max(axis=2)
    move = k * np.exp2(np.floor(np.log2(np.maximum(blk, 1e-30))) - 7) / np.sqrt(128.0)
    ulp = np.exp2(np.floor(np.log2(np.maximum(np.abs(b), 1e-30))) - 7)
    tol = ulp + np.repeat(move, 128, axis=1)
    err = np.abs(a - b)
    d = ulp_diff_bf16(dev_bits, ref_bits)
    rep = dict(max_ulp=int(d.max()) if d.size else 0, frac_ulp=float((d > 0).mean()) if d.size else 0.0,
               worst=float((err / tol).max()) if d.size else 0.0)
    assert rep["worst"] <= 1.0 and rep["frac_ulp"] <= frac, f"{what}: {rep}"
    return rep


def code_mismatch_report(gpu_packed: np.ndarray, ref: dict, bits: int) -> dict:
    """Compare packed codes with the oracle's; classify mismatches.

    A mismatch is a tie flip when the codes differ by one and the oracle's pre-rounding
    value t lies within 1e-3 of the half-integer between them (fp32 reassociation inside
    the MFMA can move t by a few ulps)."""
    g = O.unpack_rowplanar(gpu_packed, bits).astype(np.int32)
    r = ref["codes_unpacked"].astype(np.int32)
    mism = g != r
    n = mism.sum()
    t = ref["t"]
    near_tie = np.abs(np.abs(t - np.floor(t)) - 0.5) < 1e-3
    tie = mism & (np.abs(g - r) == 1) & (near_tie | (t < 0) | (t > (1 << bits) - 1))
    return dict(n=int(g.size), mismatches=int(n), tie_flips=int(tie.sum()), other=int((mism & ~tie).sum()),
                frac=float(n) / g.size)


def assert_codes(gpu_packed, ref, bits, budget=TIE_BUDGET, what="codes"):
    rep = code_mismatch_report(np.asarray(gpu_packed), ref, bits)
    assert rep["frac"] <= budget, f"{what}: {rep}"
    return rep


def assert_fp_close(gpu_bits: np.ndarray, ref_f64: np.ndarray, what: str,
                    max_abs=MAX_ABS, rel_l2=REL_L2) -> dict:
    """Fused output (bf16 bits) vs the float64 oracle result: max-abs and rel-L2 bars, plus
    the bf16 ulp-flip count against the once-rounded oracle."""
    g = O.bf16_to_f32(gpu_bits).astype(np.float64)
    ref_rounded = O.bf16_to_f32(O.round_out(ref_f64)).astype(np.float64)
    diff = g - ref_rounded
    mx = float(np.abs(diff).max()) if diff.size else 0.0
    den = float(np.linalg.norm(ref_rounded)) or 1.0
    rl2 = float(np.linalg.norm(diff)) / den
    flips = int((ulp_diff_bf16(gpu_bits, O.round_out(ref_f64)) > 0).sum())
    rep = dict(max_abs=mx, rel_l2=rl2, ulp_flips=flips, n=int(g.size))
    assert mx <= max_abs and rl2 <= rel_l2, f"{what}: {rep}"
    return rep
