"""Pins the CPU oracle (oracle/lrq_oracle.py) before it is trusted as the parity checker.

Each oracle function is checked against something independent of its own formula:
  * known answers built by construction (tests/golden/known_answers.json, written by
    tests/golden/make_known_answers.py from integer arithmetic alone);
  * library routines: torch's bf16 / fp16 conversions, torch.matmul, torch.topk,
    torch.kthvalue, Tensor.to_sparse, autograd, and the aten backward functions (silu_backward, gelu_backward(approximate='tanh'),
    _softmax_backward_data), evaluated in float64 on the CPU;
  * an independent torch-eager restatement of the reference's torch forms
    (low_rank_extraction_fuse_compression_quantization.py:153-171,
    low_rank_extraction_fuse_decompression_dequantization.py:155-165), and the invariant
    decode(encode(x)) == the naive round trip (low_rank_kernel_accuracy_test.py:6-16);
  * closed forms and brute force: exact rational fma, H128 H128 = 128 I, nearest-level search
    for the group quantiser, quantiser invariants.
No GPU is needed.
"""

from __future__ import annotations

import json
import math
from fractions import Fraction
from pathlib import Path

import numpy as np
import pytest
import torch

import oracle as O

GOLD = json.loads((Path(__file__).resolve().parent / "golden" / "known_answers.json").read_text())


def _bf(a) -> np.ndarray:
    return np.asarray(a, dtype=np.uint16)


# ------------------------------------------------------------------ rounding helpers
def test_bf16_round_matches_torch():
    g = torch.Generator().manual_seed(0)
    x = torch.cat([torch.randn(20000, generator=g) * 10, torch.randn(2000, generator=g) * 1e-39,
                   torch.tensor([0.0, -0.0, 1.0, 1.00390625, 1.01171875, 65504.0, 3e38, float("inf"), -float("inf")])])
    # exact midpoints between bf16 neighbours (ties to even)
    mids = (torch.arange(1, 200, dtype=torch.int32) << 16) + 0x8000
    x = torch.cat([x, mids.view(torch.float32)])
    ref = x.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(O.bf16_round(x.numpy()), ref)


def test_f16_sat_matches_torch_in_range():
    g = torch.Generator().manual_seed(1)
    x = torch.randn(10000, generator=g) * 1000
    assert np.array_equal(O.f16_sat(x.numpy()).view(np.uint16), x.to(torch.float16).numpy().view(np.uint16))
    assert O.f16_sat(np.array([1e6, -1e6], np.float32)).tolist() == [65504.0, -65504.0]


def test_fma32_is_correctly_rounded():
    rng = np.random.default_rng(2)
    a = rng.standard_normal(3000).astype(np.float32)
    b = rng.standard_normal(3000).astype(np.float32)
    c = (rng.standard_normal(3000) * 4).astype(np.float32)
    # cases whose exact value sits on a float32 midpoint (the TwoSum correction decides)
    one = np.float32(1.0)
    eps = np.float32(2.0 ** -24)
    a = np.concatenate([a, [one, one, np.float32(3.0)]]).astype(np.float32)
    b = np.concatenate([b, [one + 2 * eps, one - eps, np.float32(1 + 2 ** -22)]]).astype(np.float32)
    c = np.concatenate([c, [np.float32(2 ** -23), np.float32(-(2 ** -25)), np.float32(-3.0)]]).astype(np.float32)
    got = O.fma32(a, b, c)
    for i in range(a.size):
        exact = Fraction(float(a[i])) * Fraction(float(b[i])) + Fraction(float(c[i]))
        r = np.float32(float(exact))  # nearest double, then float32 ...
        # ... corrected to the nearest float32 of the exact rational (ties to even)
        cands = [np.nextafter(r, np.float32(-np.inf)), r, np.nextafter(r, np.float32(np.inf))]
        dist = [abs(Fraction(float(v)) - exact) for v in cands]
        best = min(dist)
        near = [v for v, d in zip(cands, dist) if d == best]
        want = near[0] if len(near) == 1 else [v for v in near if (np.float32(v).view(np.uint32) & 1) == 0][0]
        assert got[i] == want, (i, a[i], b[i], c[i], got[i], want)


def test_rcp32_correct_for_fp16_values():
    h = np.arange(1, 0x7C00, dtype=np.uint16).view(np.float16).astype(np.float32)
    r = O.rcp32(h)
    exact = 1.0 / h.astype(np.float64)
    # correctly rounded: within half an ulp
    ulp = np.abs(np.nextafter(r, np.float32(np.inf)) - r).astype(np.float64)
    assert np.all(np.abs(r.astype(np.float64) - exact) <= ulp / 2 * (1 + 1e-12))


# ------------------------------------------------------------------ packing
@pytest.mark.parametrize("case", GOLD["rowplanar"], ids=lambda c: f"b{c['bits']}")
def test_rowplanar_known_answers(case):
    codes = np.array(case["codes"], dtype=np.uint8)
    packed = O.pack_rowplanar(codes, case["bits"])
    assert packed.tolist() == case["packed"]
    assert np.array_equal(O.unpack_rowplanar(packed, case["bits"]), codes)


def _torch_pack(q: torch.Tensor, bits: int) -> torch.Tensor:
    """Independent restatement of the reference's packing loop: plane i (columns
    [i*N/E, (i+1)*N/E)) shifted by bits*i and or-ed into one byte per column."""
    e = 8 // bits
    n = q.shape[-1] // e
    out = torch.zeros(q.shape[:-1] + (n,), dtype=torch.int16)
    for i in range(e):
        out |= q[..., i * n:(i + 1) * n].to(torch.int16) << (bits * i)
    return out.to(torch.uint8)


@pytest.mark.parametrize("bits", [1, 2, 4, 8])
def test_rowplanar_matches_reference_packing(bits):
    g = torch.Generator().manual_seed(bits)
    q = torch.randint(0, 1 << bits, (3, 5, 64), generator=g, dtype=torch.int16)
    assert np.array_equal(O.pack_rowplanar(q.numpy().astype(np.uint8), bits), _torch_pack(q, bits).numpy())


# ------------------------------------------------------------------ legacy forms
@pytest.mark.parametrize("case", GOLD["legacy_encode"], ids=lambda c: c["name"])
def test_legacy_encode_known_answers(case):
    M, N, K = case["M"], case["N"], case["K"]
    l = np.zeros((M, K), np.uint16)
    r = np.zeros((K, N), np.uint16)
    x = _bf(case["x"])[None]
    s = _bf(case["s"])[None]
    o, q = O.legacy_encode(l, r, x, s, case["bits"], case["tau"])
    assert q[0].tolist() == case["q"]
    assert o[0].tolist() == case["o"]


def test_legacy_decode_known_answer():
    case = GOLD["legacy_decode"][0]
    M, N, K = case["M"], case["N"], case["K"]
    xh = O.legacy_decode(np.zeros((M, K), np.uint16), np.zeros((K, N), np.uint16),
                         np.array(case["q"], np.uint8)[None], _bf(case["o"])[None], _bf(case["s"])[None], case["bits"])
    assert xh[0].tolist() == case["x_hat"]


def _torch_legacy_encode(l, r, x, s, bits, outlier):
    """The reference's torch encode form restated with CPU bf16 tensors."""
    x = x - l @ r
    keep = torch.abs(x) > outlier
    o = x * keep
    x = x - o
    q = torch.clamp(torch.round(x / s.unsqueeze(-2)), min=-2 ** (bits - 1), max=2 ** (bits - 1) - 1)
    return o, _torch_pack(q.to(torch.int16) + 2 ** (bits - 1), bits)


def _torch_legacy_decode(l, r, q, o, s, bits):
    """The reference's torch decode form restated with CPU tensors (q as int8)."""
    e = 8 // bits
    n = q.shape[-1]
    mask = (1 << bits) - 1
    x = torch.empty(q.shape[:-1] + (n * e,), dtype=torch.int8)
    qq = q.to(torch.int8)
    for i in range(e):
        x[..., i * n:(i + 1) * n] = ((qq & mask) - 2 ** (bits - 1)).to(torch.int8)
        qq = qq >> bits
    return x * s.unsqueeze(-2) + o + l @ r


@pytest.mark.parametrize("bits", [2, 4, 8])
def test_legacy_forms_match_torch_restatement(bits):
    g = torch.Generator().manual_seed(40 + bits)
    B, M, N, K = 2, 24, 64, 16
    l = (torch.randn(M, K, generator=g) * 0.5).to(torch.bfloat16)
    r = (torch.randn(K, N, generator=g) * 0.5).to(torch.bfloat16)
    x = (torch.randn(B, M, N, generator=g) * 2).to(torch.bfloat16)
    s = (0.05 + 0.3 * torch.rand(B, N, generator=g)).to(torch.bfloat16)
    bits16 = lambda t: t.contiguous().view(torch.int16).numpy().view(np.uint16)  # noqa: E731
    o_ref, q_ref = _torch_legacy_encode(l, r, x, s, bits, 5.0)
    o, q = O.legacy_encode(bits16(l), bits16(r), bits16(x), bits16(s), bits, 5.0)
    # torch's CPU GEMM sums in its own order; the oracle rounds the exact sum: allow rare flips
    assert (q != q_ref.numpy()).mean() <= 2e-3
    nz = (O.bf16_to_f32(o) != 0) | (o_ref.float().numpy() != 0)
    assert (o[nz] != bits16(o_ref)[nz]).mean() <= 2e-3
    xh_ref = _torch_legacy_decode(l, r, torch.from_numpy(q), o_ref, s, bits)
    xh = O.legacy_decode(bits16(l), bits16(r), q, bits16(o_ref), bits16(s), bits)
    assert (xh != bits16(xh_ref)).mean() <= 2e-3


def test_legacy_roundtrip_equals_naive():
    """decode(encode(x)) == the naive unpacked round trip, exactly (same l @ r)."""
    rng = np.random.default_rng(5)
    B, M, N, K, bits = 2, 16, 64, 16, 4
    l = O.bf16_round(rng.standard_normal((M, K)).astype(np.float32) * 0.5)
    r = O.bf16_round(rng.standard_normal((K, N)).astype(np.float32) * 0.5)
    x = O.bf16_round(rng.standard_normal((B, M, N)).astype(np.float32) * 3)
    s = O.bf16_round((0.05 + 0.3 * rng.random((1, N))).astype(np.float32))
    o, q = O.legacy_encode(l, r, x, s, bits, 5.0)
    assert np.array_equal(O.legacy_decode(l, r, q, o, s, bits), O.naive_roundtrip(l, r, x, s, bits, 5.0))


def test_lowrank_add_matches_torch():
    g = torch.Generator().manual_seed(6)
    l = torch.randn(16, 16, generator=g).to(torch.bfloat16)
    r = torch.randn(16, 96, generator=g).to(torch.bfloat16)
    x = torch.randn(2, 16, 96, generator=g).to(torch.bfloat16)
    bits16 = lambda t: t.contiguous().view(torch.int16).numpy().view(np.uint16)  # noqa: E731
    ref = bits16(x + l @ r)
    assert (O.lowrank_add(bits16(l), bits16(r), bits16(x)) != ref).mean() <= 2e-3


# ------------------------------------------------------------------ group quantiser
def test_group_quantiser_known_answer():
    case = GOLD["group_ramp"]
    r = np.array(case["r"], dtype=np.float32)
    codes, scale, zero, _ = O.quant_groups(r, case["bits"], case["group"])
    assert codes.tolist() == case["codes"]
    assert scale.astype(np.float64).tolist() == case["scale"]
    assert zero.astype(np.float64).tolist() == case["zero"]
    d = O.dequant_groups(codes, scale, zero, case["group"])
    assert np.array_equal(d, r)  # both groups are on their quantisation grids


@pytest.mark.parametrize("bits,group", [(4, 64), (8, 128), (4, 128)])
def test_group_quantiser_invariants_and_brute_force(bits, group):
    rng = np.random.default_rng(bits * 1000 + group)
    r = (rng.standard_normal((40, 4 * group)) * rng.uniform(0.01, 30, (40, 1))).astype(np.float32)
    codes, scale, zero, t = O.quant_groups(r, bits, group)
    qmax = (1 << bits) - 1
    assert codes.max() <= qmax
    cg = codes.reshape(40, -1, group)
    # min and max of every group land on the end codes (up to fp16 rounding of scale/zero)
    assert (cg.min(axis=-1) <= 1).all() and (cg.max(axis=-1) >= qmax - 1).all()
    d = O.dequant_groups(codes, scale, zero, group).astype(np.float64)
    sc = np.repeat(scale.astype(np.float64), group, axis=-1)
    err = np.abs(d - r)
    assert (err <= sc * 0.5 * (1 + 2e-3) + np.abs(r) * 2e-6).all()
    # brute force: the code is the nearest level of zero + k*scale unless the value is
    # within rounding noise of a midpoint or outside the representable range
    z = np.repeat(zero.astype(np.float64), group, axis=-1)
    levels = np.clip(np.rint((r - z) / sc), 0, qmax)
    near_mid = np.abs(np.abs((r - z) / sc - np.floor((r - z) / sc)) - 0.5) < 1e-3
    ok = (levels == codes) | near_mid
    assert ok.mean() == 1.0


def test_group_quantiser_planted_error_is_caught():
    """A quantiser with a transposed zero-point sign fails the dequant error bound."""
    rng = np.random.default_rng(9)
    r = rng.standard_normal((8, 128)).astype(np.float32) + 3
    codes, scale, zero, _ = O.quant_groups(r, 4, 64)
    bad = O.dequant_groups(codes, scale, (-zero.astype(np.float32)).astype(np.float16), 64)
    sc = np.repeat(scale.astype(np.float64), 64, axis=-1)
    assert not (np.abs(bad - r) <= sc * 0.5 * 1.002).all()


# ------------------------------------------------------------------ WHT-128
def test_sylvester_closed_form():
    h = O.sylvester(128)
    assert np.array_equal(h @ h, 128 * np.eye(128, dtype=np.int64))
    o, k = np.meshgrid(np.arange(128), np.arange(128), indexing="ij")
    par = np.vectorize(lambda v: bin(v).count("1") & 1)(o & k)
    assert np.array_equal(h, np.where(par == 1, -1, 1))


@pytest.mark.parametrize("case", GOLD["wht_unit"], ids=lambda c: f"e{c['k']}")
def test_wht_unit_vectors(case):
    x = np.zeros((1, 256), np.uint16)
    x[0, 128 + case["k"]] = 0x3F80  # 1.0 in the second block
    y = O.wht128_bf16(x)
    assert (y[0, :128] == 0).all()
    assert y[0, 128:].tolist() == case["y"]


def test_wht_chunks_partition_the_block():
    cols = np.concatenate(O.wht128_chunks())
    assert sorted(cols.tolist()) == list(range(128))


def test_wht_matches_matrix_product_and_inverts():
    rng = np.random.default_rng(3)
    x = O.bf16_to_f32(O.bf16_round(rng.standard_normal((6, 512)).astype(np.float32)))
    y = O.wht128_rows(x).astype(np.float64)
    h = O.sylvester(128).astype(np.float64) / math.sqrt(128)
    ref = (x.astype(np.float64).reshape(6, 4, 128) @ h).reshape(6, 512)
    assert np.abs(y - ref).max() <= 4e-7 * np.abs(ref).max()
    assert np.allclose(np.linalg.norm(y, axis=1), np.linalg.norm(x, axis=1), rtol=1e-6)
    back = O.wht128_rows(y.astype(np.float32))
    assert np.abs(back - x).max() <= 1e-6 * np.abs(x).max()


# ------------------------------------------------------------------ projection / group encode
def test_projection_matches_torch_matmul():
    rng = np.random.default_rng(4)
    y = O.bf16_to_f32(O.bf16_round(rng.standard_normal((20, 256)).astype(np.float32)))
    v = O.bf16_round(np.linalg.qr(rng.standard_normal((256, 16)))[0].astype(np.float32))
    l_bits, l32 = O.projection(y, v)
    ref = (torch.from_numpy(y).double() @ torch.from_numpy(O.bf16_to_f32(v)).double()).float().numpy()
    assert np.array_equal(l32, ref)
    assert np.array_equal(l_bits, O.bf16_round(ref))


@pytest.mark.parametrize("rank,hadamard", [(16, False), (0, False), (16, True)])
def test_group_roundtrip_error_bound(rank, hadamard):
    rng = np.random.default_rng(10 + rank)
    M, N = 12, 512
    x = O.bf16_round(rng.standard_normal((M, N)).astype(np.float32))
    v = O.bf16_round(np.linalg.qr(rng.standard_normal((N, 16)))[0].astype(np.float32)) if rank else None
    enc = O.encode(x, v, 4, 64, hadamard=hadamard)
    y = O.reconstruct_f32(enc["L"], v, enc["codes"], enc["scale"], enc["zero"], 4, 64)
    # before the inverse rotation the reconstruction is within scale/2 of the rotated input
    sc = np.repeat(enc["scale"].astype(np.float64), 64, axis=-1)
    assert (np.abs(y.astype(np.float64) - enc["Y"]) <= sc * 0.5 * 1.002 + np.abs(enc["Y"]) * 2e-6).all()
    xh = O.bf16_to_f32(O.decode(enc["L"], v, enc["codes"], enc["scale"], enc["zero"], 4, 64, hadamard=hadamard))
    x32 = O.bf16_to_f32(x)
    assert np.linalg.norm(xh - x32) / np.linalg.norm(x32) < 0.15


def test_outlier_channels_and_topk():
    rng = np.random.default_rng(7)
    x = rng.standard_normal((64, 256)).astype(np.float32)
    chans = rng.choice(256, 5, replace=False)
    x[:, chans] *= 50
    xb = O.bf16_round(x)
    cm = O.colmax_abs(xb)
    ref = torch.from_numpy(np.abs(O.bf16_to_f32(xb))).amax(dim=0).numpy()
    assert np.array_equal(cm, ref)
    idx = O.topk_channels(cm, 5)
    assert np.array_equal(idx, np.sort(torch.topk(torch.from_numpy(cm), 5).indices.numpy()))
    assert sorted(idx.tolist()) == sorted(chans.tolist())
    enc = O.encode(xb, None, 8, 128, outlier_idx=idx)
    assert np.array_equal(enc["side"], O.bf16_to_f32(xb)[:, idx].astype(np.float16))
    d = O.decode(None, None, enc["codes"], enc["scale"], enc["zero"], 8, 128, side=enc["side"], idx=idx)
    assert np.array_equal(O.bf16_to_f32(d)[:, idx], enc["side"].astype(np.float32))


# ------------------------------------------------------------------ consumers
def test_consumers_match_aten_backward_functions():
    g = torch.Generator().manual_seed(8)
    x = torch.randn(4, 300, generator=g, dtype=torch.float64) * 3
    dy = torch.randn(4, 300, generator=g, dtype=torch.float64) * 0.02
    assert np.allclose(O.silu_bwd(x.numpy(), dy.numpy()), torch.ops.aten.silu_backward(dy, x).numpy(),
                       rtol=1e-12, atol=1e-15)
    assert np.allclose(O.gelu_bwd(x.numpy(), dy.numpy()),
                       torch.ops.aten.gelu_backward(dy, x, approximate="tanh").numpy(), rtol=1e-12, atol=1e-15)
    p = torch.softmax(torch.randn(4, 300, generator=g, dtype=torch.float64), dim=-1)
    assert np.allclose(O.softmax_bwd(p.numpy(), dy.numpy()),
                       torch._softmax_backward_data(dy, p, -1, torch.float64).numpy(), rtol=1e-12, atol=1e-18)
    a = torch.randn(300, 7, generator=g, dtype=torch.float64)
    assert np.allclose(O.gemm(x.numpy(), a.numpy()), (x @ a).numpy(), rtol=1e-12)
    assert np.array_equal(O.mul(x.numpy(), dy.numpy()), (x * dy).numpy())


def test_gemm_t_is_the_lora_factor_gradient():
    """gemm_t(x, dy B^T) is dL/dA of y = x W^T + (x A) B under upstream dy, as torch autograd
    computes it (a transposed operand or a dropped factor fails here)."""
    g = torch.Generator().manual_seed(9)
    x = torch.randn(37, 64, generator=g, dtype=torch.float64)
    w = torch.randn(48, 64, generator=g, dtype=torch.float64)
    a = torch.randn(64, 16, generator=g, dtype=torch.float64, requires_grad=True)
    b = torch.randn(16, 48, generator=g, dtype=torch.float64)
    dy = torch.randn(37, 48, generator=g, dtype=torch.float64)
    y = x @ w.T + (x @ a) @ b
    (da,) = torch.autograd.grad(y, a, dy)
    got = O.gemm_t(x.numpy(), (dy @ b.T).numpy())
    assert got.shape == (64, 16)
    assert np.allclose(got, da.numpy(), rtol=1e-12, atol=1e-12)


def test_round_out_is_single_rounding():
    v = np.array([1.0 + 2 ** -9, 1.0 + 3 * 2 ** -9, -2.5e-3], np.float64)
    assert np.array_equal(O.round_out(v), O.bf16_round(v.astype(np.float32)))


def test_legacy_residual_matches_torch_restatement():
    """legacy_residual = the reference's `x - l @ r` on CPU bf16 tensors (rare GEMM-order flips)."""
    g = torch.Generator().manual_seed(44)
    l = (torch.randn(24, 16, generator=g) * 0.5).to(torch.bfloat16)
    r = (torch.randn(16, 64, generator=g) * 0.5).to(torch.bfloat16)
    x = (torch.randn(24, 64, generator=g) * 2).to(torch.bfloat16)
    b16 = lambda t: t.contiguous().view(torch.int16).numpy().view(np.uint16)  # noqa: E731
    got = O.legacy_residual(b16(l), b16(r), b16(x))
    assert (got != b16(x - l @ r)).mean() <= 2e-3
    # the encode's residual: with threshold 0 every nonzero residual is an outlier, o == xr
    o, _ = O.legacy_encode(b16(l), b16(r), b16(x)[None], np.full((1, 64), 0x3F80, np.uint16), 8, 0.0)
    nz = (got & 0x7FFF) != 0
    assert np.array_equal(o[0][nz], got[nz])


def test_kth_smallest_abs_matches_torch_kthvalue():
    g = torch.Generator().manual_seed(45)
    x = (torch.randn(37, 53, generator=g) * 3).to(torch.bfloat16)
    x[0, :5] = 0.0
    x[1, :3] = -0.0
    x[2, :9] = 1.5  # ties
    xb = x.contiguous().view(torch.int16).numpy().view(np.uint16)
    n = x.numel()
    for k in (1, 7, n // 2, int(n * 0.99), n):
        ref = torch.kthvalue(x.flatten().abs().to(torch.float32), k).values.item()
        assert O.kth_smallest_abs(xb, k) == np.float32(ref), k


@pytest.mark.parametrize("shape", [(2, 5, 70), (40, 33), (300,)])
def test_to_coo_matches_torch_to_sparse(shape):
    g = torch.Generator().manual_seed(46)
    x = torch.randn(shape, generator=g)
    x = torch.where(torch.rand(shape, generator=g) < 0.9, torch.zeros(shape), x)
    x.view(-1)[::7] = -0.0  # negative zeros are not entries
    x = x.to(torch.bfloat16)
    xb = x.contiguous().view(torch.int16).numpy().view(np.uint16)
    idx, vals = O.to_coo(xb)
    sp = x.to_sparse()
    assert sp.is_coalesced()
    assert np.array_equal(idx, sp.indices().numpy())
    assert np.array_equal(vals, sp.values().contiguous().view(torch.int16).numpy().view(np.uint16))


# ------------------------------------------------------------------ the torch-eager CPU baseline
@pytest.mark.parametrize("rows,hidden,rank,bits,group,hadamard,k", [
    (64, 1024, 16, 4, 64, False, 0),
    (64, 1024, 32, 8, 128, True, 0),
    (64, 1024, 0, 8, 128, False, 9),
    (128, 2048, 16, 4, 64, False, 5),
    (64, 1024, 16, 4, 64, True, 7),
])
def test_torch_restatement_matches_oracle(pkg, rows, hidden, rank, bits, group, hadamard, k):
    """oracle/lrq_torch.py (the CPU baseline bench.py times) computes what lrq_oracle computes:
    L within one bf16 ulp on <= 1% of entries (fp32 vs exact sums), codes equal given that L
    except for <= 1e-4 rounding flips, qparams equal, and the decode within the floating-point
    bar (bf16-exact where no rotation reorders the sums)."""
    from oracle import lrq_torch as T
    from parity import assert_fp_close, bits16, ulp_diff_bf16
    x = pkg.inputs.activation(rows, hidden, 8, 20.0, seed=3)
    V = pkg.inputs.basis(hidden, rank, seed=3) if rank else None
    idx = (torch.tensor(sorted(np.random.default_rng(0).choice(hidden, k, replace=False)), dtype=torch.int32)
           if k else None)
    e = T.encode(x, V, bits, group, hadamard, idx)
    vb = bits16(V) if rank else None
    ib = idx.numpy() if k else None
    if rank:
        d = ulp_diff_bf16(bits16(e["L"]), O.encode(bits16(x), vb, bits, group, hadamard=hadamard, outlier_idx=ib)["L"])
        assert d.max() <= (64 if hadamard else 1) and (d > 0).mean() <= 1e-2
    ref = O.encode(bits16(x), vb, bits, group, hadamard=hadamard, outlier_idx=ib,
                   l_override=bits16(e["L"]) if rank else None)
    cu = O.unpack_rowplanar(e["codes"].numpy(), bits).astype(np.int32)
    cr = ref["codes_unpacked"].astype(np.int32)
    assert np.abs(cu - cr).max() <= 1 and (cu != cr).mean() <= 1e-4
    assert np.array_equal(e["scale"].numpy(), ref["scale"]) and np.array_equal(e["zero"].numpy(), ref["zero"])
    if k:
        assert np.array_equal(e["side"].numpy(), ref["side"])
    xh = T.decode(e, V, bits, group, hadamard)
    ro = O.reconstruct_f32(bits16(e["L"]) if rank else None, vb, e["codes"].numpy(), e["scale"].numpy(),
                           e["zero"].numpy(), bits, group, hadamard=hadamard, side=ref["side"], idx=ib)
    assert_fp_close(bits16(xh), ro.astype(np.float64), "torch decode")
    if not hadamard:
        assert (ulp_diff_bf16(bits16(xh), O.round_out(ro)) > 0).mean() <= 1e-5


def test_torch_restatement_consumers_and_legacy(pkg):
    """The torch-eager consumers and the reference's torch legacy forms against lrq_oracle."""
    from oracle import lrq_torch as T
    from parity import assert_fp_close, bits16, ulp_diff_bf16
    x = pkg.inputs.activation(64, 1024, 0, 1.0, seed=4)
    dy = pkg.inputs.gradient((64, 1024), 0.02, seed=4)
    xf, dyf = O.bf16_to_f32(bits16(x)), O.bf16_to_f32(bits16(dy))
    assert_fp_close(bits16(T.silu_bwd(x, dy)), O.silu_bwd(xf, dyf), "torch silu")
    assert_fp_close(bits16(T.gelu_bwd(x, dy)), O.gelu_bwd(xf, dyf), "torch gelu")
    p = pkg.inputs.softmax_probs((64, 1024), seed=4)
    assert_fp_close(bits16(T.softmax_bwd(p, dy)), O.softmax_bwd(O.bf16_to_f32(bits16(p)), dyf), "torch softmax")
    cfg = pkg.inputs.CONFIGS["legacy"]
    ops = pkg.inputs.legacy_operands(cfg)
    l, r, s = ops["l"][:256], ops["r"][:, :1024], ops["s"][:, :1024]
    xl = pkg.inputs.activation(256, 1024, 8, 20.0, seed=1)[None]
    for bits in (2, 4, 8):
        o, q = T.legacy_encode(l, r, xl, s, bits, 2.0)
        ro, rq = O.legacy_encode(bits16(l), bits16(r), bits16(xl), bits16(s), bits, 2.0)
        assert np.array_equal(q.numpy(), rq)
        assert np.array_equal(O.bf16_to_f32(bits16(o)), O.bf16_to_f32(ro))  # equal values (+-0 alike)
        xh = T.legacy_decode(l, r, q, o, s, bits)
        d = ulp_diff_bf16(bits16(xh), O.legacy_decode(bits16(l), bits16(r), rq, ro, bits16(s), bits))
        assert d.max() <= 1 and (d > 0).mean() <= 1e-4


@pytest.mark.parametrize("rank", [0, 16])
def test_outliers_with_rotation_compose(pkg, rank):
    """Outlier channels on the rotated format: the channels leave before the rotation.  Pinned
    by composition: the encode equals the rotated encode of x with those columns zeroed (plus
    the fp16 side columns of the original x), and the decode equals the rotated decode of that
    encode with the side columns written over its idx columns afterwards.  Dropping the zeroing,
    or substituting before the rotation, fails one of these."""
    x = pkg.inputs.activation(48, 1024, 6, 40.0, seed=11)
    xb = O.bf16_round(x.float().numpy())
    vb = O.bf16_round(pkg.inputs.basis(1024, rank, seed=11).float().numpy()) if rank else None
    idx = O.topk_channels(O.colmax_abs(xb), 6)
    e = O.encode(xb, vb, 4, 64, hadamard=True, outlier_idx=idx)
    xm = xb.copy()
    xm[:, idx] = 0
    e0 = O.encode(xm, vb, 4, 64, hadamard=True)
    assert np.array_equal(e["codes"], e0["codes"])
    assert np.array_equal(e["scale"].view(np.uint16), e0["scale"].view(np.uint16))
    if rank:
        assert np.array_equal(e["L"], e0["L"])
    assert np.array_equal(e["side"], O.bf16_to_f32(xb[:, idx]).astype(np.float16))
    d = O.decode(e["L"], vb, e["codes"], e["scale"], e["zero"], 4, 64, hadamard=True, side=e["side"], idx=idx)
    d0 = O.decode(e0["L"], vb, e0["codes"], e0["scale"], e0["zero"], 4, 64, hadamard=True)
    rest = np.setdiff1d(np.arange(1024), idx)
    assert np.array_equal(d[:, rest], d0[:, rest])
    assert np.array_equal(d[:, idx], O.bf16_round(e["side"].astype(np.float32)))
    # the outlier channels come back exactly where fp16 holds them; the rest at the quantiser's scale
    xf = O.bf16_to_f32(xb).astype(np.float64)
    err = O.bf16_to_f32(d).astype(np.float64) - xf
    assert np.abs(err[:, idx]).max() <= 2.0 ** -11 * np.abs(xf[:, idx]).max()
    assert np.linalg.norm(err) / np.linalg.norm(xf) < 0.1
