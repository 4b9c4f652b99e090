"""GPU parity of the blockwise WHT-128 rotation (N4) and of the rotated compressed format
(config 4 recipe at reduced rows).  The rotation sums in the order the oracle defines
(wht128_rows), so its bf16 output must match bit for bit; the rotated encode is checked like
the plain one (codes conditional on the device's L, then end to end), and decode against the
oracle's decode of the device's codes.
"""

import importlib

import numpy as np
import pytest
import torch

import oracle as O
from parity import TIE_BUDGET, assert_codes, assert_fp_close, assert_rotated_close, bits16, f16, ulp_diff_bf16

pytestmark = pytest.mark.gpu


# 512-column slabs (row-persistent kernel, several row blocks per workgroup at 20000 rows)
# and widths that take the per-block kernel (128, 640)
@pytest.mark.parametrize("rows,n", [(50, 1024), (16, 5120), (20000, 512), (3, 128), (35, 640)])
def test_wht128_bitexact(pkg, dev, rows, n):
    g = torch.Generator().manual_seed(rows + n)
    x = (torch.randn(rows, n, generator=g) * 3).to(torch.bfloat16)
    xb = bits16(x)
    y = pkg.wht128(x.to(dev))
    torch.cuda.synchronize()
    ref = O.wht128_bf16(xb)
    # The oracle rounds once per 32-term MFMA step; on gfx950 that model holds for all but a
    # few elements in ten million (20000 x 512: 2 elements, 1 ulp of bf16), so the bar is
    # <= 1 ulp on at most 1e-6 of the elements (and bit-exact at the smaller sizes).
    d = ulp_diff_bf16(bits16(y), ref)
    assert d.max() <= 1 and (d > 0).mean() <= 1e-6, (int(d.max()), int((d > 0).sum()))
    # in place gives the same bits as out of place, and the rotation undoes itself to within
    # bf16 rounding
    xd = x.to(dev).clone()
    pkg.wht128(xd, out=xd)
    assert np.array_equal(bits16(xd), bits16(y))
    back = bits16(pkg.wht128(y))
    d2 = ulp_diff_bf16(back, O.wht128_bf16(bits16(y)))
    assert d2.max() <= 1 and (d2 > 0).mean() <= 1e-6
    err = np.abs(O.bf16_to_f32(back) - O.bf16_to_f32(xb))
    assert err.max() <= 0.05 * np.abs(O.bf16_to_f32(xb)).max()


# 2560 columns: 20 units, so the decode's last workgroup of a row holds 4 of its 8 units (the
# rotation blocks past them are left alone)
@pytest.mark.parametrize("rows,n", [(64, 5120), (100, 2560)])
def test_rotated_format_c4_recipe(pkg, dev, rows, n):
    """Config 4: X [rows, 5120], 16 outlier channels x30, rotation, rank 16, int4/g64."""
    rank = 16
    print("[c4] inputs", flush=True)
    x = pkg.inputs.activation(rows, n, 16, 30.0, seed=4)
    V = pkg.inputs.basis(n, rank, seed=4)
    xb, vb = bits16(x), bits16(V)
    c = pkg.encode(x.to(dev), V.to(dev), bits=4, group_size=64, hadamard=True)
    torch.cuda.synchronize()
    lg = bits16(c.L)
    ref_full = O.encode(xb, vb, 4, 64, hadamard=True)
    d = ulp_diff_bf16(lg, ref_full["L"])
    assert d.max() <= 1 and (d > 0).sum() <= max(2, 1e-3 * d.size)
    ref = O.encode(xb, vb, 4, 64, hadamard=True, l_override=lg)
    codes = c.codes.cpu().numpy()
    rep = assert_codes(codes, ref, 4, what="rotated codes | device L")
    assert_codes(codes, ref_full, 4, what="rotated codes end-to-end")
    print(f"[c4] codes {rep}", flush=True)
    xh = pkg.decode(c)
    torch.cuda.synchronize()
    ref_xh = O.decode(lg, vb, codes, f16(c.scale), f16(c.zero), 4, 64, hadamard=True)
    flips = int((bits16(xh) != ref_xh).sum())
    assert flips <= TIE_BUDGET * ref_xh.size + 1, flips
    # round-trip error of the rotated format stays at the quantiser's scale
    x32 = O.bf16_to_f32(xb).astype(np.float64)
    e = O.bf16_to_f32(bits16(xh)).astype(np.float64) - x32
    rel = np.linalg.norm(e) / np.linalg.norm(x32)
    print(f"[c4] round-trip rel-L2 {rel:.4f}", flush=True)
    assert rel < 0.1
    # consumers on the rotated format compose decode + dense op
    dy = pkg.inputs.gradient((rows, n), 0.02, seed=4)
    out = pkg.silu_backward_compressed(c, dy.to(dev))
    xhf = O.bf16_to_f32(ref_xh)
    assert_fp_close(bits16(out), O.silu_bwd(xhf, O.bf16_to_f32(bits16(dy))), "rotated SiLU bwd")


@pytest.mark.parametrize("rows,n,rank,bits,group,op", [
    (37, 5120, 16, 4, 64, "silu"),    # config 4's format: fused in the row decode (EpiRot), ragged rows
    (64, 2560, 0, 4, 64, "gelu"),     # rank 0; 20 units (a workgroup with 4 of its 8 units)
    (40, 2048, 32, 4, 64, "mul"),     # rank 32 (two blocks in flight)
    (30, 2048, 16, 8, 128, "silu"),   # int8 / g128: fused (4 units per workgroup)
    (52, 4096, 0, 8, 128, "gelu"),    # int8 / g128 at rank 0, config 3's width
    (24, 2048, 16, 4, 64, "softmax"), # softmax: fused two-sweep kernel over rotation blocks
    (40, 2048, 32, 4, 64, "softmax"), # rank 32
    (33, 4096, 16, 8, 128, "softmax"),  # int8 / g128
    (24, 384, 16, 4, 64, "softmax"),  # planes of 192 columns: decode, then the dense backward in place
])
def test_rotated_consumers(pkg, dev, rows, n, rank, bits, group, op):
    """Consumers on the rotated format: bit-identical to the dense op on the device's own decode
    (the same rotation code and the same elementwise formula; the fused softmax sums its rows in
    another order, so it is held to the floating-point bar there), and within the floating-point
    bar of the oracle's rotated decode followed by the op in float64."""
    print(f"[rot consumer] rows={rows} n={n} rank={rank} int{bits}/g{group} {op}", flush=True)
    x = pkg.inputs.activation(rows, n, 8, 20.0, seed=n + rank)
    if op == "softmax":
        x = torch.softmax(x.float() / 8.0, dim=-1).to(torch.bfloat16)
    V = pkg.inputs.basis(n, rank, seed=3) if rank else None
    c = pkg.encode(x.to(dev), V.to(dev) if V is not None else None, bits=bits, group_size=group, hadamard=True)
    y = pkg.inputs.gradient((rows, n), 0.02, seed=rows)
    fn = {"silu": pkg.silu_backward_compressed, "gelu": pkg.gelu_backward_compressed,
          "mul": pkg.mul_compressed, "softmax": pkg.softmax_backward_compressed}[op]
    out = fn(c, y.to(dev))
    xh = pkg.decode(c)
    torch.cuda.synchronize()
    xd = O.bf16_to_f32(bits16(xh))
    yf = O.bf16_to_f32(bits16(y))
    ref_dev = {"silu": O.silu_bwd, "gelu": O.gelu_bwd, "mul": O.mul, "softmax": O.softmax_bwd}[op](xd, yf)
    assert_fp_close(bits16(out), ref_dev, f"rotated {op} vs the device decode")
    # the very same fp32 formula on the same x_hat: the library's dense kernels on the decode
    dense = {"silu": pkg.triton_silu_backward, "gelu": pkg.triton_gelu_backward, "mul": pkg.triton_hadamard,
             "softmax": pkg.triton_softmax_backward}[op](xh, y.to(dev))
    torch.cuda.synchronize()
    if op == "softmax" and (n // (8 // bits)) % 128 == 0:
        assert_fp_close(bits16(out), O.softmax_bwd(O.bf16_to_f32(bits16(xh)), yf), "fused rotated softmax vs dense")
    else:
        assert np.array_equal(bits16(out), bits16(dense))
    ref_xh = O.decode(bits16(c.L) if rank else None, bits16(V) if rank else None, c.codes.cpu().numpy(),
                      f16(c.scale), f16(c.zero), bits, group, hadamard=True)
    # rank 32 reconstructs with MFMA fp32 sums that can sit a step from the oracle's, and the
    # rotation spreads such a difference over 128 outputs
    print(f"[rot consumer] decode {assert_rotated_close(bits16(xh), ref_xh, 'rotated decode')}", flush=True)
    ref = {"silu": O.silu_bwd, "gelu": O.gelu_bwd, "mul": O.mul, "softmax": O.softmax_bwd}[op](
        O.bf16_to_f32(ref_xh), yf)
    rep = assert_fp_close(bits16(out), ref, f"rotated {op} vs the oracle")
    print(f"[rot consumer] {rep}", flush=True)


@pytest.mark.parametrize("bits,group,rank", [(4, 64, 16), (4, 64, 32), (8, 128, 16), (4, 128, 0), (8, 64, 0)])
def test_rotated_softmax_reads_the_decoded_p(pkg, dev, bits, group, rank):
    """The fused rotated softmax backward with dP one-hot per row (dP[r, k_r] = 1): the row sum is
    P[r, k_r] exactly and dS[r, c] = bf16(fp32(P[r, c] (0 - P[r, k_r]))) (fp32(1 - P) at c = k_r), so
    dS computed in float32 from the rotated decode's P must match bit for bit: the kernel's P is
    the decode's.  In place (dS over dP) gives the same bits."""
    import ctypes
    L = importlib.import_module("triton-kernel-test_amd._lib")
    lib = L.load()
    print(f"[rot softmax P] int{bits}/g{group} rank={rank}", flush=True)
    rows, n = 70, 2048
    x = torch.softmax(pkg.inputs.activation(rows, n, 8, 20.0, seed=bits * group).float() / 8.0, dim=-1)
    x = x.to(torch.bfloat16)
    V = pkg.inputs.basis(n, rank, seed=11) if rank else None
    c = pkg.encode(x.to(dev), V.to(dev) if V is not None else None, bits=bits, group_size=group, hadamard=True)
    k = np.random.default_rng(rows + rank).integers(0, n, rows)
    dp = torch.zeros(rows, n, dtype=torch.bfloat16)
    dp[torch.arange(rows), torch.as_tensor(k)] = 1.0
    out = pkg.softmax_backward_compressed(c, dp.to(dev))
    xh = pkg.decode(c)
    buf = dp.to(dev)
    d = c.descriptor()
    sp = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    pb = ctypes.c_void_p(buf.data_ptr())
    st = lib.lrq_softmax_bwd(ctypes.byref(d), pb, n, pb, n, sp)
    torch.cuda.synchronize()
    assert st == 0 and torch.equal(buf, out)
    P = O.bf16_to_f32(bits16(xh)).astype(np.float32)
    pk = P[np.arange(rows), k]
    dv = np.zeros_like(P)
    dv[np.arange(rows), k] = 1.0
    want = P * (dv - pk[:, None])  # float32 operations, as the kernel's
    assert np.array_equal(bits16(out), O.round_out(want.astype(np.float64)))


@pytest.mark.parametrize("rows,n,rank,bits,group,fused", [
    (37, 5120, 16, 4, 64, True),     # fused rotated row kernel: dx written over dy gives the same bits
    (30, 2048, 16, 8, 128, True),    # int8 / g128: fused too (4 units per workgroup)
    (30, 2048, 16, 4, 128, False),   # int4 / g128: decode then dense op, so an aliasing call is refused
])
def test_rotated_consumer_in_place(pkg, dev, rows, n, rank, bits, group, fused):
    """dx == dy through the C ABI on the rotated format: the fused kernel reads each dy element
    before writing that dx element, so in place equals out of place; the decode-then-dense form
    would overwrite dy first, so it returns LRQ_ERR_UNSUPPORTED and leaves dy untouched."""
    import ctypes
    L = importlib.import_module("triton-kernel-test_amd._lib")
    lib = L.load()
    print(f"[rot in place] rows={rows} n={n} int{bits}/g{group}", flush=True)
    x = pkg.inputs.activation(rows, n, 8, 20.0, seed=n + 7)
    V = pkg.inputs.basis(n, rank, seed=3)
    c = pkg.encode(x.to(dev), V.to(dev), bits=bits, group_size=group, hadamard=True)
    dy = pkg.inputs.gradient((rows, n), 0.02, seed=rows + 1).to(dev)
    ref = pkg.silu_backward_compressed(c, dy)
    buf = dy.clone()
    d = c.descriptor()
    sp = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    p = ctypes.c_void_p(buf.data_ptr())
    st = lib.lrq_silu_bwd(ctypes.byref(d), p, n, p, n, sp)
    torch.cuda.synchronize()
    if fused:
        assert st == 0 and torch.equal(buf, ref)
    else:
        assert st == L.LRQ_ERR_UNSUPPORTED and torch.equal(buf, dy)


@pytest.mark.parametrize("rows,n,rank,n_out,out_dtype,bits,group", [
    (64, 5120, 16, 16, torch.float32, 4, 64),     # config 4's format
    (37, 2560, 0, 32, torch.bfloat16, 4, 64),     # 20 units: the last step holds 4 of 8; ragged rows
    (40, 2048, 16, 16, torch.float32, 8, 128),    # int8 / g128: one rotation block per unit
    (30, 2048, 16, 32, torch.float32, 4, 128),    # int4 / g128, n = 32: two blocks per unit, no prefetch
    (50, 1024, 0, 16, torch.float32, 8, 64),      # int8 / g64: half a block per unit, four row blocks per workgroup
])
def test_rotated_dequant_gemm(pkg, dev, rows, n, rank, n_out, out_dtype, bits, group):
    """x_hat @ A on the rotated format, fused: against the float64 product on the device's rotated
    decode (the kernel's in-register rotation sums what the decode's does, so the x_hat is the
    same) within the fp32 accumulation bound, and against the oracle's rotated decode within the
    floating-point bar."""
    print(f"[rot gemm] rows={rows} n={n} rank={rank} n_out={n_out} {out_dtype} int{bits}/g{group}", flush=True)
    x = pkg.inputs.activation(rows, n, 8, 20.0, seed=n + n_out)
    V = pkg.inputs.basis(n, rank, seed=5) if rank else None
    gen = torch.Generator().manual_seed(n_out)
    a = (torch.randn(n, n_out, generator=gen) / np.sqrt(n)).to(torch.bfloat16)
    c = pkg.encode(x.to(dev), V.to(dev) if V is not None else None, bits=bits, group_size=group, hadamard=True)
    out = pkg.dequant_gemm(c, a.to(dev), out_dtype=out_dtype)
    xh = pkg.decode(c)
    torch.cuda.synchronize()
    xd = O.bf16_to_f32(bits16(xh)).astype(np.float64)
    af = O.bf16_to_f32(bits16(a)).astype(np.float64)
    ref = xd @ af
    bound = 1e-5 * (np.abs(xd) @ np.abs(af)) + 1e-9
    if out_dtype == torch.float32:
        got = out.cpu().numpy().astype(np.float64)
        err = np.abs(got - ref)
        assert (err <= bound).all(), (float(err.max()), float((err / bound).max()))
    else:
        got = O.bf16_to_f32(bits16(out)).astype(np.float64)
        ulp = np.exp2(np.floor(np.log2(np.maximum(np.abs(ref), 1e-30))) - 7)
        assert (np.abs(got - ref) <= ulp + bound).all()
    ref_xh = O.decode(bits16(c.L) if rank else None, bits16(V) if rank else None, c.codes.cpu().numpy(),
                      f16(c.scale), f16(c.zero), bits, group, hadamard=True)
    ref_o = O.gemm(O.bf16_to_f32(ref_xh), af)
    if out_dtype == torch.float32:
        rel = np.linalg.norm(got - ref_o) / np.linalg.norm(ref_o)
        assert rel <= 1e-3, rel
    else:
        assert_fp_close(bits16(out), ref_o, "rotated dequant gemm bf16 vs the oracle")


@pytest.mark.parametrize("bits,group,rank,n_out", [
    (4, 64, 16, 16), (4, 64, 32, 32), (8, 128, 16, 16), (4, 128, 0, 32), (8, 64, 0, 16)])
def test_rotated_dequant_gemm_reads_the_decoded_x_hat(pkg, dev, bits, group, rank, n_out):
    """With A one-hot (column k selects input column c_k), x_hat A is column k = x_hat[:, c_k]
    exactly (one product by 1, the rest exact zeros), so the in-register rotation's x_hat is
    compared bit for bit with the rotated decode's, n_out columns spread over planes and blocks."""
    print(f"[rot gemm x_hat] int{bits}/g{group} rank={rank} n={n_out}", flush=True)
    rows, n = 70, 2048
    x = pkg.inputs.activation(rows, n, 8, 20.0, seed=bits + group + rank)
    V = pkg.inputs.basis(n, rank, seed=8) if rank else None
    c = pkg.encode(x.to(dev), V.to(dev) if V is not None else None, bits=bits, group_size=group, hadamard=True)
    sel = np.sort(np.random.default_rng(n_out + bits).choice(n, n_out, replace=False))
    a = torch.zeros(n, n_out, dtype=torch.bfloat16)
    a[torch.as_tensor(sel), torch.arange(n_out)] = 1.0
    out = pkg.dequant_gemm(c, a.to(dev), out_dtype=torch.float32)
    xh = pkg.decode(c)
    torch.cuda.synchronize()
    want = O.bf16_to_f32(bits16(xh))[:, sel].astype(np.float32)
    got = out.cpu().numpy().reshape(rows, n_out)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), int((got != want).sum())


def test_rotated_dequant_gemm_straddling_planes(pkg, dev):
    """int4/g64 at 384 columns: planes of 192 columns, so rotation blocks straddle the planes and
    the fused GEMM refuses (the decode still works through its separate rotation pass)."""
    x = pkg.inputs.activation(16, 384, 0, 1.0, seed=1)
    c = pkg.encode(x.to(dev), None, bits=4, group_size=64, hadamard=True)
    with pytest.raises(ValueError, match="lrq_dequant_gemm"):
        pkg.dequant_gemm(c, torch.zeros(384, 16, dtype=torch.bfloat16, device=dev))


@pytest.mark.parametrize("rows,n,rank,bits,group,k", [
    (64, 5120, 16, 4, 64, 16),    # config 4 with its 16 outlier channels kept as side columns
    (40, 2048, 0, 4, 64, 9),      # rank 0
    (30, 2048, 32, 4, 64, 5),     # rank 32
    (36, 2048, 16, 8, 128, 12),   # int8 / g128
    (20, 2048, 16, 4, 64, 100),   # more side columns than the row decode stages
])
def test_outliers_with_rotation(pkg, dev, rows, n, rank, bits, group, k):
    """Outlier channels on the rotated format: they leave X before the rotation (fp16 side
    columns of the original values) and return after the inverse rotation.  Encode against
    the oracle (L within an ulp, codes given the device L), decode within the rotated bar with the
    side columns exact, a fused consumer bit-identical to the dense op on the device decode, and
    the dequant-GEMM (up to 64 channels) within the fp32 accumulation bound."""
    print(f"[outliers+rot] rows={rows} n={n} rank={rank} int{bits}/g{group} k={k}", flush=True)
    x = pkg.inputs.activation(rows, n, k, 40.0, seed=k + rank)
    V = pkg.inputs.basis(n, rank, seed=k) if rank else None
    xb = bits16(x)
    vb = bits16(V) if rank else None
    idx = O.topk_channels(O.colmax_abs(xb), k)
    c = pkg.encode(x.to(dev), V.to(dev) if V is not None else None, bits=bits, group_size=group, hadamard=True,
                   outlier_idx=torch.as_tensor(idx, dtype=torch.int32, device=dev))
    torch.cuda.synchronize()
    assert np.array_equal(f16(c.side).view(np.uint16), O.bf16_to_f32(xb[:, idx]).astype(np.float16).view(np.uint16))
    ref_full = O.encode(xb, vb, bits, group, hadamard=True, outlier_idx=idx)
    if rank:
        lg = bits16(c.L)
        d = ulp_diff_bf16(lg, ref_full["L"])
        assert d.max() <= 1 and (d > 0).sum() <= max(2, 1e-3 * d.size)
    ref = O.encode(xb, vb, bits, group, hadamard=True, outlier_idx=idx, l_override=bits16(c.L) if rank else None)
    codes = c.codes.cpu().numpy()
    rep = assert_codes(codes, ref, bits, what="rotated codes with side columns | device L")
    print(f"[outliers+rot] codes {rep}", flush=True)
    xh = pkg.decode(c)
    dy = pkg.inputs.gradient((rows, n), 0.02, seed=k)
    dx = pkg.silu_backward_compressed(c, dy.to(dev))
    dense = pkg.triton_silu_backward(xh, dy.to(dev))
    torch.cuda.synchronize()
    ref_xh = O.decode(bits16(c.L) if rank else None, vb, codes, f16(c.scale), f16(c.zero), bits, group,
                      hadamard=True, side=f16(c.side), idx=idx)
    assert np.array_equal(bits16(xh)[:, idx], ref_xh[:, idx])
    print(f"[outliers+rot] decode {assert_rotated_close(bits16(xh), ref_xh, 'rotated decode with side columns')}",
          flush=True)
    assert np.array_equal(bits16(dx), bits16(dense))
    if k <= 64:
        a = (torch.randn(n, 16, generator=torch.Generator().manual_seed(k)) / np.sqrt(n)).to(torch.bfloat16)
        out = pkg.dequant_gemm(c, a.to(dev))
        torch.cuda.synchronize()
        xd = O.bf16_to_f32(bits16(xh)).astype(np.float64)
        af = O.bf16_to_f32(bits16(a)).astype(np.float64)
        err = np.abs(out.cpu().numpy().astype(np.float64) - xd @ af)
        bound = 1e-5 * (np.abs(xd) @ np.abs(af)) + 1e-9
        assert (err <= bound).all(), float((err / bound).max())
    # x_hat^T g: the side columns' output rows come from the side values, the rest from the
    # rotated x_hat (any channel count)
    gm = (torch.randn(rows, 16, generator=torch.Generator().manual_seed(k + 1)) * 0.05).to(torch.bfloat16)
    da = pkg.dequant_gemm_t(c, gm.to(dev))
    torch.cuda.synchronize()
    xd = O.bf16_to_f32(bits16(xh)).astype(np.float64)
    gf = O.bf16_to_f32(bits16(gm)).astype(np.float64)
    err = np.abs(da.cpu().numpy().astype(np.float64) - xd.T @ gf)
    bound = 1e-5 * (np.abs(xd).T @ np.abs(gf)) + 1e-9
    assert (err <= bound).all(), float((err / bound).max())


@pytest.mark.parametrize("rows,n,rank,n_out,out_dtype,bits,group", [
    (64, 5120, 16, 16, torch.float32, 4, 64),     # config 4's format
    (37, 2560, 0, 32, torch.bfloat16, 4, 64),     # n = 32: one plane per wave; ragged rows
    (40, 2048, 16, 16, torch.float32, 8, 128),    # int8 / g128: one unit per rotation block
    (300, 2048, 32, 32, torch.float32, 4, 64),    # rank 32, several blocks per wave
    (30, 2048, 16, 32, torch.float32, 4, 128),    # int4 / g128
    (50, 1024, 0, 16, torch.float32, 8, 64),      # int8 / g64: two units per rotation block
    (7995, 2048, 16, 16, torch.float32, 4, 64),   # 16 row groups of 32 blocks (XCD-aware mapping), ragged ends
    (3000, 4096, 16, 32, torch.float32, 4, 64),   # fewer blocks than whole chunks for 256 workgroups
])
def test_rotated_dequant_gemm_t(pkg, dev, rows, n, rank, n_out, out_dtype, bits, group):
    """x_hat^T @ g on the rotated format, fused (the rotation's transposed MFMA form leaves x_hat
    with the rows along the registers): against the float64 product on the device's rotated
    decode within the fp32 accumulation bound (one bf16 rounding more for bf16 out), and against
    the oracle's rotated decode within the floating-point bar; the allocation-free entry point
    gives the same bits."""
    print(f"[rot gemm_t] rows={rows} n={n} rank={rank} n_out={n_out} {out_dtype} int{bits}/g{group}", flush=True)
    x = pkg.inputs.activation(rows, n, 8, 20.0, seed=n + n_out + 1)
    V = pkg.inputs.basis(n, rank, seed=6) if rank else None
    gm = (torch.randn(rows, n_out, generator=torch.Generator().manual_seed(rows)) * 0.05).to(torch.bfloat16)
    c = pkg.encode(x.to(dev), V.to(dev) if V is not None else None, bits=bits, group_size=group, hadamard=True)
    out = pkg.dequant_gemm_t(c, gm.to(dev), out_dtype=out_dtype)
    out2 = torch.empty_like(out)
    pkg.dequant_gemm_t_noalloc(c, gm.to(dev), out2)
    xh = pkg.decode(c)
    torch.cuda.synchronize()
    assert torch.equal(out, out2)
    xd = O.bf16_to_f32(bits16(xh)).astype(np.float64)
    gf = O.bf16_to_f32(bits16(gm)).astype(np.float64)
    ref = xd.T @ gf
    bound = 1e-5 * (np.abs(xd).T @ np.abs(gf)) + 1e-9
    if out_dtype == torch.float32:
        got = out.cpu().numpy().astype(np.float64)
        err = np.abs(got - ref)
        assert (err <= bound).all(), (float(err.max()), float((err / bound).max()))
    else:
        got = O.bf16_to_f32(bits16(out)).astype(np.float64)
        ulp = np.exp2(np.floor(np.log2(np.maximum(np.abs(ref), 1e-30))) - 7)
        assert (np.abs(got - ref) <= ulp + bound).all()
    ref_xh = O.decode(bits16(c.L) if rank else None, bits16(V) if rank else None, c.codes.cpu().numpy(),
                      f16(c.scale), f16(c.zero), bits, group, hadamard=True)
    ref_o = O.gemm_t(O.bf16_to_f32(ref_xh), O.bf16_to_f32(bits16(gm)))
    if out_dtype == torch.float32:
        rel = np.linalg.norm(got - ref_o) / np.linalg.norm(ref_o)
        assert rel <= 1e-3, rel
    else:
        assert_fp_close(bits16(out), ref_o, "rotated dequant gemm_t bf16 vs the oracle")


@pytest.mark.parametrize("bits,group,rank,n_out", [
    (4, 64, 16, 16), (4, 64, 32, 32), (8, 128, 16, 16), (4, 128, 0, 32), (8, 64, 0, 32)])
def test_rotated_dequant_gemm_t_reads_the_decoded_x_hat(pkg, dev, bits, group, rank, n_out):
    """With g one-hot (column k selects row r_k), x_hat^T g is column k = x_hat[r_k, :] exactly
    (one product by 1, the rest exact zeros), so the fused kernel's rotated x_hat is compared
    bit for bit with the rotated decode's, every column of n_out rows."""
    print(f"[rot gemm_t x_hat] int{bits}/g{group} rank={rank} n={n_out}", flush=True)
    rows, n = 80, 2048
    x = pkg.inputs.activation(rows, n, 8, 20.0, seed=bits + group)
    V = pkg.inputs.basis(n, rank, seed=7) if rank else None
    c = pkg.encode(x.to(dev), V.to(dev) if V is not None else None, bits=bits, group_size=group, hadamard=True)
    sel = np.sort(np.random.default_rng(n_out + rank).choice(rows, n_out, replace=False))
    gm = torch.zeros(rows, n_out, dtype=torch.bfloat16)
    gm[torch.as_tensor(sel), torch.arange(n_out)] = 1.0
    out = pkg.dequant_gemm_t(c, gm.to(dev))
    xh = pkg.decode(c)
    torch.cuda.synchronize()
    want = O.bf16_to_f32(bits16(xh))[sel, :].T
    got = out.cpu().numpy()
    assert np.array_equal(got.view(np.uint32), want.astype(np.float32).view(np.uint32)), \
        int((got != want).sum())


def test_rotated_lora_grads(pkg, dev):
    """lora_grads on the rotated format (the two fused products): the same bits as dequant_gemm
    and dequant_gemm_t called one by one."""
    rows, n = 200, 4096
    x = pkg.inputs.activation(rows, n, 8, 20.0, seed=9)
    V = pkg.inputs.basis(n, 16, seed=9)
    c = pkg.encode(x.to(dev), V.to(dev), bits=4, group_size=64, hadamard=True)
    a = (torch.randn(n, 16, generator=torch.Generator().manual_seed(1)) / np.sqrt(n)).to(torch.bfloat16).to(dev)
    gm = (torch.randn(rows, 16, generator=torch.Generator().manual_seed(2)) * 0.05).to(torch.bfloat16).to(dev)
    xa, da = pkg.lora_grads(c, a, gm)
    xa1 = pkg.dequant_gemm(c, a, out_dtype=torch.bfloat16).reshape(-1, 16)
    da1 = pkg.dequant_gemm_t(c, gm, out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert torch.equal(xa, xa1) and torch.equal(da, da1)
