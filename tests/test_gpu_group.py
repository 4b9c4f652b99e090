"""GPU parity of the group-mode path (north-star format) against the CPU oracle.

Inputs are drawn on the CPU (identical bits on both sides) and moved to the device.  Each
check is done twice where the projection is involved: conditionally on the device's L
(isolates the quantiser, which must match bit-exactly) and end-to-end against the oracle's
own L (tie-flip budget 1e-4 of codes).
"""

import numpy as np
import pytest
import torch

import oracle as O
from parity import (assert_codes, assert_decode_close, assert_fp_close, assert_projection_close, bits16,
                    code_mismatch_report, f16, from_bits, ulp_diff_bf16)

pytestmark = pytest.mark.gpu


def _np_inputs(x, V):
    xb = bits16(x)
    vb = bits16(V) if V is not None else None
    return xb, vb


def _check_encode(pkg, dev, x, V, bits, group, twopass=False, outlier_idx=None):
    xb, vb = _np_inputs(x, V)
    idx_t = None if outlier_idx is None else torch.as_tensor(outlier_idx, dtype=torch.int32, device=dev)
    c = pkg.encode(x.to(dev), V.to(dev) if V is not None else None, bits=bits, group_size=group,
                   outlier_idx=idx_t, _twopass=twopass)
    torch.cuda.synchronize()
    rep = {}
    if V is not None:
        lg = bits16(c.L)
        ref_full = O.encode(xb, vb, bits, group, outlier_idx=outlier_idx)
        d = ulp_diff_bf16(lg, ref_full["L"])
        rep["L_flips"] = int((d > 0).sum())
        assert d.max() <= 1, f"L differs by {d.max()} ulps"
        assert rep["L_flips"] <= max(2, 1e-3 * d.size), rep
        ref = O.encode(xb, vb, bits, group, outlier_idx=outlier_idx, l_override=lg)
    else:
        ref_full = ref = O.encode(xb, None, bits, group, outlier_idx=outlier_idx)
    codes = c.codes.cpu().numpy()
    rep["cond"] = assert_codes(codes, ref, bits, what="codes | device L")
    sc, ze = f16(c.scale), f16(c.zero)
    rep["scale_mism"] = int((sc.view(np.uint16) != ref["scale"].view(np.uint16)).sum())
    rep["zero_mism"] = int((ze.view(np.uint16) != ref["zero"].view(np.uint16)).sum())
    assert rep["scale_mism"] <= 1e-4 * sc.size + 1 and rep["zero_mism"] <= 1e-4 * ze.size + 1, rep
    rep["full"] = assert_codes(codes, ref_full, bits, what="codes end-to-end")
    if outlier_idx is not None:
        side = f16(c.side)
        assert np.array_equal(side.view(np.uint16), ref["side"].view(np.uint16))
    return c, ref, rep


FORMATS = [
    # (rows, hidden, rank, bits, group)
    (100, 4096, 16, 4, 64),    # fused single pass (8 waves x 8 chunks), ragged rows
    (64, 2048, 16, 4, 64),     # fused (4 x 8)
    (48, 5120, 16, 4, 64),     # fused (8 x 10)
    (37, 1536, 16, 4, 64),     # two-pass (no single-pass instantiation)
    (64, 4096, 32, 4, 64),     # rank 32 (column-slab two-pass)
    (72, 11008, 32, 4, 64),    # rank 32 at config 2's width: 6 slabs, the last one partial
    (40, 2048, 16, 4, 128),
    (33, 2048, 16, 8, 64),
    (64, 1024, 16, 8, 128),
    (50, 2048, 0, 4, 64),      # rank 0
    (50, 1024, 0, 8, 128),
]


@pytest.mark.parametrize("rows,hidden,rank,bits,group", FORMATS)
def test_encode_decode_formats(pkg, dev, rows, hidden, rank, bits, group):
    print(f"[encode/decode] rows={rows} hidden={hidden} rank={rank} bits={bits} group={group}", flush=True)
    x = pkg.inputs.activation(rows, hidden, n_outlier=4, outlier_scale=20.0, seed=rows + hidden)
    V = pkg.inputs.basis(hidden, rank, seed=7) if rank else None
    c, ref, rep = _check_encode(pkg, dev, x, V, bits, group)
    # decode of the device's compressed data vs the oracle's decode of the same data
    xh = pkg.decode(c)
    torch.cuda.synchronize()
    ref_xh = O.decode(bits16(c.L) if rank else None, bits16(V) if rank else None, c.codes.cpu().numpy(),
                      f16(c.scale), f16(c.zero), bits, group)
    d = ulp_diff_bf16(bits16(xh), ref_xh)
    assert d.max() <= 1 and (d > 0).mean() <= 1e-3, (d.max(), (d > 0).mean())


@pytest.mark.parametrize("rows,hidden,rank,bits,group,k", [
    (100, 4096, 16, 4, 64, 41),   # row-staged single pass (4 units per wave), config 3's channel count
    (5000, 4096, 16, 4, 64, 8),   # several row blocks per workgroup, ragged
    (64, 2048, 16, 4, 64, 9),     # row-staged, 2 units per wave (slice staged through registers)
    (64, 4096, 32, 4, 64, 41),    # rank 32: the column-slab passes
    (72, 11008, 32, 4, 64, 20),   # config 2's format
    (40, 4096, 16, 8, 128, 41),   # int8 / g128 with rank 16: the slab passes
    (33, 1536, 16, 4, 64, 5),     # the slab passes (no single-pass kernel for 12 units)
])
def test_outlier_channels_with_low_rank(pkg, dev, rows, hidden, rank, bits, group, k):
    """Outlier channels combined with the rank-r extraction: the channels are zeroed before the
    projection and kept as fp16 side columns (low_rank_extraction_fuse_compression_quantization.py:66-82
    subtracts l@r and splits outliers in one kernel).  Encode, decode and a fused consumer
    against the oracle."""
    print(f"[outliers+rank] rows={rows} hidden={hidden} rank={rank} int{bits}/g{group} k={k}", flush=True)
    x = pkg.inputs.activation(rows, hidden, n_outlier=k, outlier_scale=50.0, seed=rows + k)
    V = pkg.inputs.basis(hidden, rank, seed=k)
    idx = O.topk_channels(O.colmax_abs(bits16(x)), k)
    c, ref, rep = _check_encode(pkg, dev, x, V, bits, group, outlier_idx=idx)
    print(f"[outliers+rank] {rep}", flush=True)
    xh = pkg.decode(c)
    dy = pkg.inputs.gradient((rows, hidden), 0.02, seed=k)
    dx = pkg.silu_backward_compressed(c, dy.to(dev))
    torch.cuda.synchronize()
    ref_xh = O.decode(bits16(c.L), bits16(V), c.codes.cpu().numpy(), f16(c.scale), f16(c.zero), bits, group,
                      side=f16(c.side), idx=idx)
    print(f"[outliers+rank] decode {assert_decode_close(bits16(xh), ref_xh, 'decode, outliers+rank')}", flush=True)
    assert np.array_equal(bits16(xh)[:, idx], ref_xh[:, idx])  # the side columns come back exactly
    assert_fp_close(bits16(dx), O.silu_bwd(O.bf16_to_f32(ref_xh), O.bf16_to_f32(bits16(dy))), "silu, outliers+rank")


@pytest.mark.parametrize("rows,hidden,rank,bits,group,k", [
    (100, 4096, 0, 4, 64, 100),    # more side columns than the row decode stages: the tile decode
    (70, 4096, 16, 4, 64, 200),    # rank 16
    (40, 2048, 0, 8, 128, 65),     # int8 / g128, one past the row decode's limit
])
def test_many_outlier_channels(pkg, dev, rows, hidden, rank, bits, group, k):
    """More than 64 outlier channels: encode and decode (k_decode, the tile kernel) against the
    oracle, and a fused consumer on the same path."""
    print(f"[outliers>64] rows={rows} hidden={hidden} rank={rank} int{bits}/g{group} k={k}", flush=True)
    x = pkg.inputs.activation(rows, hidden, n_outlier=k, outlier_scale=50.0, seed=k)
    V = pkg.inputs.basis(hidden, rank, seed=k) if rank else None
    idx = O.topk_channels(O.colmax_abs(bits16(x)), k)
    c, ref, rep = _check_encode(pkg, dev, x, V, bits, group, outlier_idx=idx)
    xh = pkg.decode(c)
    dy = pkg.inputs.gradient((rows, hidden), 0.02, seed=k)
    dx = pkg.gelu_backward_compressed(c, dy.to(dev))
    torch.cuda.synchronize()
    ref_xh = O.decode(bits16(c.L) if rank else None, bits16(V) if rank else None, c.codes.cpu().numpy(),
                      f16(c.scale), f16(c.zero), bits, group, side=f16(c.side), idx=idx)
    print(f"[outliers>64] decode {assert_decode_close(bits16(xh), ref_xh, 'decode, >64 outliers')}", flush=True)
    assert np.array_equal(bits16(xh)[:, idx], ref_xh[:, idx])
    assert_fp_close(bits16(dx), O.gelu_bwd(O.bf16_to_f32(ref_xh), O.bf16_to_f32(bits16(dy))), "gelu, >64 outliers")


# 4100 rows: 257 row blocks, so on 256 CUs the single-pass kernels walk two blocks per
# workgroup (the next block's loads in flight) and the last block is ragged; 5120 columns take
# the tile-staged kernel, plain and rotated
@pytest.mark.parametrize("rows,hidden,rank,bits,group,hadamard", [
    (100, 4096, 16, 4, 64, False), (64, 5120, 16, 4, 64, False), (4100, 4096, 16, 4, 64, False),
    (4100, 5120, 16, 4, 64, False), (4100, 5120, 16, 4, 64, True), (37, 5120, 16, 4, 64, True)])
def test_twopass_matches_fused(pkg, dev, rows, hidden, rank, bits, group, hadamard):
    print(f"[twopass] rows={rows} hidden={hidden} hadamard={hadamard}", flush=True)
    x = pkg.inputs.activation(rows, hidden, 8, 20.0, seed=3).to(dev)
    V = pkg.inputs.basis(hidden, rank, seed=3).to(dev)
    a = pkg.encode(x, V, bits=bits, group_size=group, hadamard=hadamard)
    b = pkg.encode(x, V, bits=bits, group_size=group, hadamard=hadamard, _twopass=True)
    torch.cuda.synchronize()
    # both against the exact projection of the (rotated) activation, within their fp32
    # accumulation bound
    y = O.bf16_to_f32(bits16(pkg.wht128(x) if hadamard else x))
    vb = bits16(V)
    ra = assert_projection_close(bits16(a.L), y, vb, "fused L")
    rb = assert_projection_close(bits16(b.L), y, vb, "two-pass L")
    print(f"[twopass] L fused {ra}, two-pass {rb}", flush=True)
    dl = ulp_diff_bf16(bits16(a.L), bits16(b.L))
    same_l = (dl == 0).all(axis=1)
    print(f"[twopass] rows with the same L: {same_l.mean():.3f}", flush=True)
    assert same_l.mean() > 0.05
    # rows whose L agrees must agree bit-for-bit in codes/scales/zeros
    ca, cb = a.codes.cpu().numpy(), b.codes.cpu().numpy()
    assert np.array_equal(ca[same_l], cb[same_l])
    assert np.array_equal(f16(a.scale)[same_l].view(np.uint16), f16(b.scale)[same_l].view(np.uint16))


def test_c1_parity(pkg, dev):
    """Config 1 at full size: [2048, 4096], 8 channels x20, rank 16, int4/g64."""
    cfg = pkg.inputs.CONFIGS["c1"]
    inp = pkg.inputs.make(cfg)
    print("[c1] encode", flush=True)
    c, ref, rep = _check_encode(pkg, dev, inp["x"], inp["V"], cfg.bits, cfg.group)
    print(f"[c1] report {rep}", flush=True)
    xh = pkg.decode(c)
    torch.cuda.synchronize()
    ref_xh = O.decode(bits16(c.L), bits16(inp["V"]), c.codes.cpu().numpy(), f16(c.scale), f16(c.zero),
                      cfg.bits, cfg.group)
    d = ulp_diff_bf16(bits16(xh), ref_xh)
    assert d.max() <= 1 and (d > 0).mean() <= 1e-4, (d.max(), (d > 0).mean())
    # round-trip error bound: |x_hat - x| <= scale/2 (+ fp16/bf16 rounding slack)
    x32 = O.bf16_to_f32(bits16(inp["x"])).astype(np.float64)
    err = np.abs(O.bf16_to_f32(bits16(xh)).astype(np.float64) - x32)
    sc = np.repeat(f16(c.scale).astype(np.float64), cfg.group, axis=1)
    bound = 0.5 * sc * (1 + 1e-2) + np.abs(x32) * 2.0 ** -8 + 1e-6
    assert (err <= bound).mean() >= 0.9999, (err / bound).max()


@pytest.mark.parametrize("op", ["silu", "gelu", "mul"])
def test_fused_elementwise(pkg, dev, op):
    rows, hidden, rank = 96, 4096, 16
    print(f"[fused {op}]", flush=True)
    x = pkg.inputs.activation(rows, hidden, 8, 20.0, seed=11)
    V = pkg.inputs.basis(hidden, rank, seed=11)
    dy = pkg.inputs.gradient((rows, hidden), 0.02, seed=11)
    c = pkg.encode(x.to(dev), V.to(dev), bits=4, group_size=64)
    fn = {"silu": pkg.silu_backward_compressed, "gelu": pkg.gelu_backward_compressed,
          "mul": pkg.mul_compressed}[op]
    out = fn(c, dy.to(dev))
    torch.cuda.synchronize()
    xh = O.bf16_to_f32(O.decode(bits16(c.L), bits16(V), c.codes.cpu().numpy(), f16(c.scale), f16(c.zero), 4, 64))
    d = O.bf16_to_f32(bits16(dy))
    ref = {"silu": O.silu_bwd, "gelu": O.gelu_bwd, "mul": O.mul}[op](xh, d)
    rep = assert_fp_close(bits16(out), ref, f"fused {op}")
    print(f"[fused {op}] {rep}", flush=True)


def test_fused_silu_c2_format(pkg, dev):
    """Config 2's format (rank 32, hidden 11008, int4/g64, 172 groups per row) on a row sample:
    the fused SiLU backward against the oracle's decompress-then-op on the device's codes."""
    cfg = pkg.inputs.CONFIGS["c2"]
    rows = 80
    inp = pkg.inputs.make(cfg, rows=rows)
    print(f"[c2 silu] rows={rows} hidden={cfg.hidden} rank={cfg.rank}", flush=True)
    c = pkg.encode(inp["x"].to(dev), inp["V"].to(dev), bits=cfg.bits, group_size=cfg.group)
    out = pkg.silu_backward_compressed(c, inp["dy"].to(dev))
    torch.cuda.synchronize()
    vb = bits16(inp["V"])
    ref_enc = O.encode(bits16(inp["x"]), vb, cfg.bits, cfg.group, l_override=bits16(c.L))
    assert_codes(c.codes.cpu().numpy(), ref_enc, cfg.bits, what="c2 codes")
    xh = O.bf16_to_f32(O.decode(bits16(c.L), vb, c.codes.cpu().numpy(), f16(c.scale), f16(c.zero), cfg.bits,
                                cfg.group))
    ref = O.silu_bwd(xh, O.bf16_to_f32(bits16(inp["dy"])))
    rep = assert_fp_close(bits16(out), ref, "c2 fused silu")
    print(f"[c2 silu] {rep}", flush=True)


@pytest.mark.parametrize("rows,bits,group", [
    (96, 4, 128),    # 128-column groups: dY staged in place, 4 waves
    (96, 8, 128),    # int8 / g128: in place, 8 waves
    (5000, 8, 128),  # several row blocks per workgroup through the in-place pipeline
])
def test_fused_gelu_g128(pkg, dev, rows, bits, group):
    hidden, rank = 4096, 16
    print(f"[fused gelu g128] rows={rows} bits={bits}", flush=True)
    x = pkg.inputs.activation(rows, hidden, 8, 20.0, seed=rows)
    V = pkg.inputs.basis(hidden, rank, seed=12)
    dy = pkg.inputs.gradient((rows, hidden), 0.02, seed=rows)
    c = pkg.encode(x.to(dev), V.to(dev), bits=bits, group_size=group)
    out = pkg.gelu_backward_compressed(c, dy.to(dev))
    torch.cuda.synchronize()
    xh = O.bf16_to_f32(O.decode(bits16(c.L), bits16(V), c.codes.cpu().numpy(), f16(c.scale), f16(c.zero),
                                bits, group))
    ref = O.gelu_bwd(xh, O.bf16_to_f32(bits16(dy)))
    rep = assert_fp_close(bits16(out), ref, "fused gelu g128")
    print(f"[fused gelu g128] {rep}", flush=True)


@pytest.mark.parametrize("rows", [512, 4100])  # 4100: several row blocks per workgroup, ragged
def test_outlier_channels_c3_shape(pkg, dev, rows):
    """Config 3 recipe at reduced rows: top-41 channels by abs-max, rank 0, int8/g128, GELU bwd."""
    cfg = pkg.inputs.CONFIGS["c3"]
    inp = pkg.inputs.make(cfg, rows=rows)
    x = inp["x"]
    print("[c3] colmax/topk", flush=True)
    xd = x.to(dev)
    cm = pkg.column_absmax(xd)
    idx = pkg.topk_channels(cm, cfg.keep_channels)
    torch.cuda.synchronize()
    xb = bits16(x)
    ref_cm = O.colmax_abs(xb)
    assert np.array_equal(cm.cpu().numpy().view(np.uint32), ref_cm.view(np.uint32))
    ref_idx = O.topk_channels(ref_cm, cfg.keep_channels)
    assert np.array_equal(idx.cpu().numpy(), ref_idx)
    print("[c3] encode", flush=True)
    c, ref, rep = _check_encode(pkg, dev, x, None, cfg.bits, cfg.group, outlier_idx=ref_idx)
    print("[c3] gelu", flush=True)
    out = pkg.gelu_backward_compressed(c, inp["dy"].to(dev))
    xh_dev = pkg.decode(c)
    torch.cuda.synchronize()
    ref_xh = O.decode(None, None, c.codes.cpu().numpy(), f16(c.scale), f16(c.zero), cfg.bits, cfg.group,
                      side=f16(c.side), idx=ref_idx)
    assert np.array_equal(bits16(xh_dev), ref_xh)
    ref_out = O.gelu_bwd(O.bf16_to_f32(ref_xh), O.bf16_to_f32(bits16(inp["dy"])))
    assert_fp_close(bits16(out), ref_out, "c3 gelu")


def test_invalid_outlier_indices(pkg, dev):
    """Device-held outlier indices are not read back: an entry outside [0, N) or a repeat of an
    earlier entry becomes -1 and its side column is zero, and every other output equals the encode
    of the valid entries alone.  Host-held indices with such entries are refused."""
    rows, hidden = 64, 4096
    print("[bad idx] encode", flush=True)
    x = pkg.inputs.activation(rows, hidden, 8, 20.0, seed=77).to(dev)
    V = pkg.inputs.basis(hidden, 16, seed=77).to(dev)
    bad = torch.tensor([10, hidden + 3, 10, 77, -1], dtype=torch.int32, device=dev)
    c = pkg.encode(x, V, outlier_idx=bad)
    good = pkg.encode(x, V, outlier_idx=torch.tensor([10, 77], dtype=torch.int32, device=dev))
    torch.cuda.synchronize()
    assert c.idx.tolist() == [10, -1, -1, 77, -1]
    assert torch.all(c.side[:, [1, 2, 4]] == 0)
    assert torch.equal(c.side[:, [0, 3]], good.side)
    assert torch.equal(c.codes, good.codes) and torch.equal(c.qparams, good.qparams) and torch.equal(c.L, good.L)
    assert torch.equal(pkg.decode(c), pkg.decode(good))
    with pytest.raises(ValueError):
        pkg.encode(x, V, outlier_idx=[10, hidden])
    with pytest.raises(ValueError):
        pkg.encode(x, V, outlier_idx=[10, 10])
