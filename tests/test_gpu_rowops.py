"""GPU parity of the row-reducing consumers on the group-mode format: the fused softmax
backward (config 5 recipe, reduced rows) and the fused dequant-GEMM (R12 build shape,
reduced rows).  The reference result is decompress-then-op on the device's own compressed
representation: x_hat = bf16(oracle decode of the device codes), then the formula in
float64, rounded once (tests/parity.py bars).
"""

import ctypes

import numpy as np
import pytest
import torch

import oracle as O
from parity import assert_fp_close, bits16, f16, ulp_diff_bf16

pytestmark = pytest.mark.gpu


def _xhat(c, V, bits, group):
    vb = bits16(V) if V is not None else None
    lb = bits16(c.L) if V is not None else None
    return O.bf16_to_f32(O.decode(lb, vb, c.codes.cpu().numpy(), f16(c.scale), f16(c.zero), bits, group))


@pytest.mark.parametrize("rows,n,rank,bits,group", [
    (100, 2048, 16, 4, 64),   # config 5 row length: 16 units, one per wave
    (9000, 2048, 16, 4, 64),  # several row blocks per workgroup (the pipelined path), last block ragged
    (64, 1024, 16, 4, 64),    # 8 units
    (48, 512, 0, 4, 64),      # 4 units, rank 0
    (40, 2048, 16, 8, 128),   # int8 / g128: 16 units
])
def test_softmax_bwd_compressed(pkg, dev, rows, n, rank, bits, group):
    print(f"[softmax] rows={rows} n={n} rank={rank} bits={bits} g={group}", flush=True)
    g = torch.Generator().manual_seed(5 + n)
    logits = torch.randn(rows, n, generator=g) / np.sqrt(128.0)
    p = torch.softmax(logits, dim=-1).to(torch.bfloat16)
    dp = (torch.randn(rows, n, generator=g) * 0.02).to(torch.bfloat16)
    V = pkg.inputs.basis(n, rank, seed=7) if rank else None
    c = pkg.encode(p.to(dev), V.to(dev) if V is not None else None, bits=bits, group_size=group)
    ds = pkg.softmax_backward_compressed(c, dp.to(dev))
    torch.cuda.synchronize()
    ph = _xhat(c, V, bits, group)
    ref = O.softmax_bwd(ph, O.bf16_to_f32(bits16(dp)))
    rep = assert_fp_close(bits16(ds), ref, "fused softmax bwd", max_abs=1e-3)
    print(f"[softmax] {rep}", flush=True)


@pytest.mark.parametrize("rows,n,rank,bits,group", [
    (100, 4096, 16, 4, 64),   # 32 units: four held per wave (reference bench width, softmax_backward.py:80)
    (37, 8192, 16, 4, 64),    # 64 units, streamed unit by unit, ragged last row block
    (64, 3072, 16, 4, 64),    # 24 units: not a multiple of the waves
    (48, 1536, 0, 4, 64),     # 12 units, rank 0
    (40, 4096, 32, 4, 64),    # rank 32
    (70, 4096, 16, 8, 128),   # int8 / g128: 32 units
    (30, 4096, 16, 4, 128),   # int4 / g128 (256-column units, loaded one at a time)
    (16, 640, 16, 8, 64),     # 10 units: two waves hold two units, six hold one
    (20, 384, 16, 4, 64),     # 3 units: fewer units than waves
    (24, 3072, 16, 4, 128),   # int4 / g128, 12 units: two held per wave at most
    (50, 2048, 16, 8, 64),    # int8 / g64, 32 units held, V operands parked in LDS
])
def test_softmax_bwd_compressed_wide(pkg, dev, rows, n, rank, bits, group):
    """Rows of any width: the fused softmax backward against the oracle's decompress-then-op
    on the device's codes."""
    print(f"[softmax wide] rows={rows} n={n} rank={rank} bits={bits} g={group}", flush=True)
    g = torch.Generator().manual_seed(50 + n + rank)
    logits = torch.randn(rows, n, generator=g) / np.sqrt(128.0)
    p = torch.softmax(logits, dim=-1).to(torch.bfloat16)
    dp = (torch.randn(rows, n, generator=g) * 0.02).to(torch.bfloat16)
    V = pkg.inputs.basis(n, rank, seed=9) if rank else None
    c = pkg.encode(p.to(dev), V.to(dev) if V is not None else None, bits=bits, group_size=group)
    ds = pkg.softmax_backward_compressed(c, dp.to(dev))
    torch.cuda.synchronize()
    ph = _xhat(c, V, bits, group)
    ref = O.softmax_bwd(ph, O.bf16_to_f32(bits16(dp)))
    rep = assert_fp_close(bits16(ds), ref, "fused softmax bwd (wide)", max_abs=1e-3)
    print(f"[softmax wide] {rep}", flush=True)


@pytest.mark.parametrize("rows,hidden,rank,n_out,out_dtype,bits,group", [
    (100, 4096, 16, 32, torch.float32, 4, 64),   # R12 build shape (reduced rows), fp32 out
    (64, 4096, 16, 32, torch.bfloat16, 4, 64),   # bf16 out
    (50, 2048, 0, 16, torch.float32, 4, 64),     # rank 0, n = 16 (wave-resident kernel, 2 units per wave)
    (100, 4096, 16, 16, torch.float32, 4, 64),   # lora shape (reduced rows): wave-resident, 4 units per wave
    (37, 4096, 16, 16, torch.bfloat16, 4, 64),   # ragged last row block, bf16 out
    (60, 3072, 16, 16, torch.float32, 4, 64),    # 24 units: not a multiple of the waves (unit-walking kernel)
    (64, 1024, 16, 16, torch.float32, 4, 64),    # 8 units: wave-resident, 1 unit per wave
    (100, 2048, 16, 16, torch.float32, 8, 128),  # int8 / g128, 16 units: 2 per wave (one plane per unit)
    (100, 2048, 0, 16, torch.bfloat16, 8, 64),   # int8 / g64, 32 units: 4 per wave, rank 0
    (100, 2048, 16, 16, torch.float32, 4, 128),  # int4 / g128, 8 units: 1 per wave, two code loads per lane
    (80, 2048, 16, 32, torch.float32, 8, 64),    # int8, n = 32: the unit-walking kernel
    (70, 2048, 16, 32, torch.bfloat16, 4, 128),  # int4 / g128, n = 32: the unit-walking kernel
])
def test_dequant_gemm(pkg, dev, rows, hidden, rank, n_out, out_dtype, bits, group):
    print(f"[gemm] rows={rows} hidden={hidden} rank={rank} n={n_out} {out_dtype} int{bits}/g{group}", flush=True)
    x = pkg.inputs.activation(rows, hidden, 8, 20.0, seed=21)
    V = pkg.inputs.basis(hidden, rank, seed=21) if rank else None
    g = torch.Generator().manual_seed(22)
    a = (torch.randn(hidden, n_out, generator=g) / np.sqrt(hidden)).to(torch.bfloat16)
    c = pkg.encode(x.to(dev), V.to(dev) if V is not None else None, bits=bits, group_size=group)
    out = pkg.dequant_gemm(c, a.to(dev), out_dtype=out_dtype)
    torch.cuda.synchronize()
    xh = _xhat(c, V, bits, group)
    ref = O.gemm(xh, O.bf16_to_f32(bits16(a)))
    if out_dtype == torch.float32:
        got = out.cpu().numpy().astype(np.float64)
        rel = np.linalg.norm(got - ref) / np.linalg.norm(ref)
        assert rel <= 1e-5 and np.abs(got - ref).max() <= 1e-3, (rel, np.abs(got - ref).max())
    else:
        assert_fp_close(bits16(out), ref, "dequant gemm bf16")


@pytest.mark.parametrize("rows,hidden,rank,n_out,out_dtype,bits,group,k", [
    (100, 4096, 16, 16, torch.float32, 4, 64, 8),     # wave-resident kernel (4 units per wave)
    (37, 2048, 0, 16, torch.bfloat16, 4, 64, 33),     # wave-resident, rank 0, two side chunks, ragged rows
    (90, 3072, 16, 32, torch.float32, 4, 64, 40),     # unit-walking kernel, n = 32
    (64, 2048, 32, 16, torch.float32, 4, 64, 64),     # rank 32, the largest side count (64)
    (50, 2048, 0, 16, torch.float32, 8, 128, 5),      # int8 / g128, rank 0
    (70, 2048, 16, 16, torch.float32, 4, 128, 12),    # int4 / g128 (256-column units)
    (60, 3072, 16, 16, torch.bfloat16, 4, 128, 20),   # int4 / g128, unit-walking kernel, one unit slot
])
def test_dequant_gemm_outliers(pkg, dev, rows, hidden, rank, n_out, out_dtype, bits, group, k):
    """x_hat @ A with outlier channels (x_hat[:, idx] = bf16(side)): against the float64 product
    on the oracle's x_hat with the side columns substituted, to the bars of test_dequant_gemm."""
    print(f"[gemm outl] rows={rows} hidden={hidden} rank={rank} n={n_out} {out_dtype} int{bits}/g{group} k={k}",
          flush=True)
    x = pkg.inputs.activation(rows, hidden, n_outlier=k, outlier_scale=50.0, seed=rows + k)
    V = pkg.inputs.basis(hidden, rank, seed=k) if rank else None
    idx = O.topk_channels(O.colmax_abs(bits16(x)), k)
    gen = torch.Generator().manual_seed(k)
    a = (torch.randn(hidden, n_out, generator=gen) / np.sqrt(hidden)).to(torch.bfloat16)
    c = pkg.encode(x.to(dev), V.to(dev) if V is not None else None, bits=bits, group_size=group,
                   outlier_idx=torch.as_tensor(idx, dtype=torch.int32, device=dev))
    out = pkg.dequant_gemm(c, a.to(dev), out_dtype=out_dtype)
    torch.cuda.synchronize()
    xh = O.bf16_to_f32(O.decode(bits16(c.L) if rank else None, bits16(V) if rank else None, c.codes.cpu().numpy(),
                                f16(c.scale), f16(c.zero), bits, group, side=f16(c.side), idx=idx))
    ref = O.gemm(xh, O.bf16_to_f32(bits16(a)))
    if out_dtype == torch.float32:
        got = out.cpu().numpy().astype(np.float64)
        rel = np.linalg.norm(got - ref) / np.linalg.norm(ref)
        assert rel <= 1e-5 and np.abs(got - ref).max() <= 1e-3 * max(1.0, np.abs(ref).max()), \
            (rel, np.abs(got - ref).max())
    else:
        assert_fp_close(bits16(out), ref, "dequant gemm bf16, outliers")


def test_dequant_gemm_outlier_limit(pkg, dev):
    """More than 64 outlier channels: the fused GEMM refuses (LRQ_ERR_UNSUPPORTED), no result."""
    x = pkg.inputs.activation(32, 2048, n_outlier=65, outlier_scale=50.0, seed=4)
    idx = O.topk_channels(O.colmax_abs(bits16(x)), 65)
    c = pkg.encode(x.to(dev), None, bits=4, group_size=64,
                   outlier_idx=torch.as_tensor(idx, dtype=torch.int32, device=dev))
    a = torch.zeros(2048, 16, dtype=torch.bfloat16, device=dev)
    with pytest.raises(ValueError, match="lrq_dequant_gemm"):
        pkg.dequant_gemm(c, a)


@pytest.mark.parametrize("rows,hidden,rank,bits,group,n_out,out_dtype", [
    (100, 4096, 16, 4, 64, 16, torch.float32),     # north-star width, reduced rows
    (3000, 4096, 16, 4, 64, 16, torch.float32),    # 6 row groups of 32 blocks, ragged last group and block
    (700, 4096, 32, 4, 64, 32, torch.bfloat16),    # rank 32, n = 32, bf16 out
    (300, 2048, 16, 8, 128, 16, torch.float32),    # int8 / g128, 2 units per wave
    (200, 1024, 16, 4, 128, 32, torch.float32),    # int4 / g128: one unit per wave
    (90, 384, 0, 4, 64, 16, torch.float32),        # odd unit count (3), rank 0
    (5, 512, 0, 8, 64, 32, torch.float32),         # fewer rows than one block
])
def test_dequant_gemm_t(pkg, dev, rows, hidden, rank, bits, group, n_out, out_dtype):
    """decode(c)^T @ g against the float64 product on lrq_decode's output (the x_hat the entry
    point is defined on): fp32 out within the accumulation bound 1e-5 * (|x_hat|^T |g|) per
    entry, bf16 out within one ulp of the once-rounded result.  Against the oracle's x_hat
    (which lrq_decode matches to 1 ulp on <= 1e-3 of elements) within the floating-point bar."""
    print(f"[gemm_t] rows={rows} hidden={hidden} rank={rank} b{bits} g{group} n={n_out} {out_dtype}", flush=True)
    x = pkg.inputs.activation(rows, hidden, 8, 20.0, seed=31)
    V = pkg.inputs.basis(hidden, rank, seed=31) if rank else None
    gen = torch.Generator().manual_seed(32)
    gm = (torch.randn(rows, n_out, generator=gen) * 0.05).to(torch.bfloat16)
    c = pkg.encode(x.to(dev), V.to(dev) if V is not None else None, bits=bits, group_size=group)
    out = pkg.dequant_gemm_t(c, gm.to(dev), out_dtype=out_dtype)
    xd = O.bf16_to_f32(bits16(pkg.decode(c)))
    torch.cuda.synchronize()
    assert out.shape == (hidden, n_out)
    gf = O.bf16_to_f32(bits16(gm))
    ref = O.gemm_t(xd, gf)
    bound = 1e-5 * O.gemm_t(np.abs(xd), np.abs(gf)) + 1e-9  # fp32 accumulation
    if out_dtype == torch.float32:
        got = out.cpu().numpy().astype(np.float64)
        err = np.abs(got - ref)
        assert (err <= bound).all(), (float(err.max()), float((err / bound).max()))
        ref_o = O.gemm_t(_xhat(c, V, bits, group), gf)
        rel = np.linalg.norm(got - ref_o) / np.linalg.norm(ref_o)
        assert rel <= 1e-3, rel
    else:
        # one bf16 rounding of a sum within the accumulation bound: |got - ref| <= ulp + bound
        got = O.bf16_to_f32(bits16(out)).astype(np.float64)
        ulp = np.exp2(np.floor(np.log2(np.maximum(np.abs(ref), 1e-30))) - 7)
        err = np.abs(got - ref)
        assert (err <= ulp + bound).all(), float((err / (ulp + bound)).max())
        flips = ulp_diff_bf16(bits16(out), O.round_out(ref))
        print(f"[gemm_t] bf16 ulp flips vs once-rounded: {int((flips > 0).sum())} of {flips.size}", flush=True)
        rep = assert_fp_close(bits16(out), O.gemm_t(_xhat(c, V, bits, group), gf), "dequant gemm_t bf16",
                              max_abs=np.inf)
        print(f"[gemm_t] vs oracle x_hat {rep}", flush=True)


@pytest.mark.parametrize("rows,hidden,rank,bits,group,n_out,k,out_dtype", [
    (300, 4096, 16, 4, 64, 16, 8, torch.float32),     # lora format with its 8 channels kept
    (1000, 2048, 0, 8, 128, 32, 41, torch.bfloat16),  # config 3's channel count, bf16 out
    (70, 1024, 32, 4, 64, 16, 100, torch.float32),    # more channels than the fused GEMM takes
])
def test_dequant_gemm_t_outliers(pkg, dev, rows, hidden, rank, bits, group, n_out, k, out_dtype):
    """decode(c)^T @ g with outlier channels (output rows idx from the side columns), against the
    float64 product on lrq_decode's output within the fp32 accumulation bound (one bf16 rounding
    more for bf16 out); the allocation-free entry point gives the same bits."""
    print(f"[gemm_t outl] rows={rows} hidden={hidden} rank={rank} int{bits}/g{group} n={n_out} k={k}", flush=True)
    x = pkg.inputs.activation(rows, hidden, n_outlier=k, outlier_scale=50.0, seed=k)
    V = pkg.inputs.basis(hidden, rank, seed=k) if rank else None
    idx = O.topk_channels(O.colmax_abs(bits16(x)), k)
    gm = (torch.randn(rows, n_out, generator=torch.Generator().manual_seed(k)) * 0.05).to(torch.bfloat16)
    c = pkg.encode(x.to(dev), V.to(dev) if V is not None else None, bits=bits, group_size=group,
                   outlier_idx=torch.as_tensor(idx, dtype=torch.int32, device=dev))
    out = pkg.dequant_gemm_t(c, gm.to(dev), out_dtype=out_dtype)
    out2 = torch.empty_like(out)
    pkg.dequant_gemm_t_noalloc(c, gm.to(dev), out2)
    xd = O.bf16_to_f32(bits16(pkg.decode(c))).astype(np.float64)
    torch.cuda.synchronize()
    assert np.array_equal(bits16(out) if out_dtype == torch.bfloat16 else out.cpu().numpy(),
                          bits16(out2) if out_dtype == torch.bfloat16 else out2.cpu().numpy())
    gf = O.bf16_to_f32(bits16(gm)).astype(np.float64)
    ref = xd.T @ gf
    bound = 1e-5 * (np.abs(xd).T @ np.abs(gf)) + 1e-9
    got = out.cpu().numpy().astype(np.float64) if out_dtype == torch.float32 else \
        O.bf16_to_f32(bits16(out)).astype(np.float64)
    ulp = 0 if out_dtype == torch.float32 else np.exp2(np.floor(np.log2(np.maximum(np.abs(ref), 1e-30))) - 7)
    err = np.abs(got - ref)
    assert (err <= ulp + bound).all(), float((err / (ulp + bound)).max())


def test_dequant_gemm_t_no_rows(pkg, dev):
    """A descriptor with rows == 0 gives dA = 0 (the sum over no rows), through the C ABI."""
    import ctypes
    _lib = __import__("importlib").import_module("triton-kernel-test_amd._lib")
    x = pkg.inputs.activation(16, 512, 0, 1.0, seed=3)
    c = pkg.encode(x.to(dev), None, bits=4, group_size=64)
    t = c.descriptor()
    t.rows = 0
    assert _lib.call_raw("lrq_dequant_gemm_t_workspace", ctypes.byref(t), 16) == 0
    gm = torch.ones(16, 16, dtype=torch.bfloat16, device=dev)
    out = torch.full((512, 16), 7.0, dtype=torch.float32, device=dev)
    s = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    st = _lib.call_raw("lrq_dequant_gemm_t", ctypes.byref(t), ctypes.c_void_p(gm.data_ptr()), 16, 16,
                       ctypes.c_void_p(out.data_ptr()), 16, 1, None, 0, s)
    torch.cuda.synchronize()
    assert st == 0 and not out.any()


@pytest.mark.parametrize("rows,hidden,out_dtype", [
    (1000, 4096, torch.float32), (17, 4096, torch.float32), (300, 2048, torch.bfloat16),
    (4100, 4096, torch.float32), (600, 8192, torch.bfloat16), (64, 1536, torch.float32)])
def test_lora_grads_one_pass(pkg, dev, rows, hidden, out_dtype):
    """lora_grads: x_hat A and x_hat^T g from one pass over the codes, against the float64
    products on lrq_decode's output (fp32 out: within the fp32 accumulation bound 1e-5 * |x_hat||.|
    per entry; bf16 out: within one ulp plus that bound), and against the two separate entry
    points (dequant_gemm, dequant_gemm_t) within twice the bound.  4100 rows: 257 row blocks, row
    groups of 9 blocks; 17 rows: groups of one block, waves with none; 1536 columns: 3 column groups."""
    print(f"[lora_grads] rows={rows} hidden={hidden} {out_dtype}", flush=True)
    x = pkg.inputs.activation(rows, hidden, 8, 20.0, seed=41)
    V = pkg.inputs.basis(hidden, 16, seed=41)
    gen = torch.Generator().manual_seed(42)
    a = (torch.randn(hidden, 16, generator=gen) * 0.05).to(torch.bfloat16)
    gm = (torch.randn(rows, 16, generator=gen) * 0.05).to(torch.bfloat16)
    c = pkg.encode(x.to(dev), V.to(dev), bits=4, group_size=64)
    t = c.descriptor()
    assert pkg._lib.call_raw("lrq_lora_grads_workspace", ctypes.byref(t), 16) > 0  # the one-pass kernel
    xa, da = pkg.lora_grads(c, a.to(dev), gm.to(dev), xa_dtype=out_dtype, da_dtype=out_dtype)
    xa_s = pkg.dequant_gemm(c, a.to(dev), out_dtype=out_dtype).reshape(rows, 16)
    da_s = pkg.dequant_gemm_t(c, gm.to(dev), out_dtype=out_dtype)
    xd = O.bf16_to_f32(bits16(pkg.decode(c))).astype(np.float64)
    torch.cuda.synchronize()
    af, gf = O.bf16_to_f32(bits16(a)), O.bf16_to_f32(bits16(gm))
    checks = (("xa", xa, xa_s, O.gemm(xd, af), 1e-5 * O.gemm(np.abs(xd), np.abs(af)) + 1e-9),
              ("da", da, da_s, O.gemm_t(xd, gf), 1e-5 * O.gemm_t(np.abs(xd), np.abs(gf)) + 1e-9))
    for name, got_t, sep_t, ref, bound in checks:
        if out_dtype == torch.float32:
            got, sep = got_t.cpu().numpy().astype(np.float64), sep_t.cpu().numpy().astype(np.float64)
            ulp = 0.0
        else:
            got, sep = (O.bf16_to_f32(bits16(v)).astype(np.float64) for v in (got_t, sep_t))
            ulp = np.exp2(np.floor(np.log2(np.maximum(np.abs(ref), 1e-30))) - 7)
        err = np.abs(got - ref)
        assert (err <= ulp + bound).all(), (name, float((err / (ulp + bound)).max()))
        assert (np.abs(got - sep) <= 2 * (ulp + bound)).all(), name
        print(f"[lora_grads] {name}: worst error / bound {float((err / (ulp + bound)).max()):.3f}", flush=True)
