"""Full-size checks at BASELINE.json's shapes, through properties that do not need the CPU
oracle over the whole tensor:

  * every group's codes span [0, qmax] and the reconstruction error of every element is
    within half a quantisation step (plus the low-rank term's bf16 rounding), evaluated on
    the device with torch ops from the kernel outputs themselves;
  * a seeded row sample of the same run matches the CPU oracle bit for bit (codes given the
    device's L) — the sample is where the oracle's cost stays bounded;
  * encode -> decode -> encode is idempotent on the codes up to ties (a decoded activation
    re-encodes to the same groups);
  * fused consumers equal decode-then-op on the device.
"""

import numpy as np
import pytest
import torch

import oracle as O
from parity import assert_codes, assert_decode_close, assert_fp_close, bits16, f16

pytestmark = pytest.mark.gpu


def _codes_unpacked(c):
    """[rows, N] int codes from the row-planar bytes (device)."""
    q = c.codes
    if c.bits == 8:
        return q.to(torch.int32)
    lo = (q & 0xF).to(torch.int32)
    hi = (q >> 4).to(torch.int32)
    return torch.cat([lo, hi], dim=1)


@pytest.mark.parametrize("name", ["north_star", "c4", "c2"])
def test_fullsize_roundtrip_properties(pkg, dev, name):
    cfg = pkg.inputs.CONFIGS[name]
    print(f"[full {name}] {cfg.rows}x{cfg.hidden}", flush=True)
    x = pkg.inputs.activation(cfg.rows, cfg.hidden, cfg.n_outlier, cfg.outlier_scale, cfg.seed, dev)
    V = pkg.inputs.basis(cfg.hidden, cfg.rank, cfg.seed)
    c = pkg.encode(x, V.to(dev), bits=cfg.bits, group_size=cfg.group, hadamard=cfg.hadamard)
    xh = pkg.decode(c)
    torch.cuda.synchronize()
    G, qmax = cfg.group, (1 << cfg.bits) - 1
    codes = _codes_unpacked(c)
    cg = codes.view(cfg.rows, -1, G)
    # min / max of a group land on the end codes unless fp16 rounding moved them by one
    assert int(cg.min(dim=-1).values.max()) <= 1 and int(cg.max(dim=-1).values.min()) >= qmax - 1
    # reconstruction before the bf16 rounding is within half a step of the residual: check on
    # the rotated-domain value Y = (rotated) x, via decode's own pieces
    y = pkg.wht128(x) if cfg.hadamard else x
    lv = (c.L.float() @ V.to(dev).float().t())
    r = y.float() - lv                                            # residual (fp32; kernel rounds once)
    d = codes.float().view(cfg.rows, -1, G) * c.scale.float()[..., None] + c.zero.float()[..., None]
    err = (d.view(cfg.rows, -1) - r).abs().view(cfg.rows, -1, G)
    step = c.scale.float()[..., None]
    bound = 0.5 * step * (1 + 2e-3) + r.abs().view(cfg.rows, -1, G) * 2e-6 + 1e-6
    frac_ok = float((err <= bound).float().mean())
    print(f"[full {name}] within half-step: {frac_ok:.7f}", flush=True)
    assert frac_ok >= 1 - 1e-6
    # decode error relative to the input stays at the quantiser's level: every element of
    # x_hat - x is within half its group's step (plus the bf16 rounding of x_hat, and of the
    # rotation for the rotated format), so the relative L2 error is bounded by those steps
    rel = float((xh.float() - x.float()).norm() / x.float().norm())
    half = (0.5 * step * (1 + 2e-3)).expand(-1, -1, G).reshape(cfg.rows, -1)
    slack = x.float().abs() * 2.0 ** -7 + 1e-6
    rel_bound = float((half + slack).norm() / x.float().norm())
    print(f"[full {name}] round-trip rel-L2 {rel:.4f} (bound {rel_bound:.4f})", flush=True)
    assert rel <= rel_bound
    # re-encode the decoded activation: same codes up to ties
    c2 = pkg.encode(xh, V.to(dev), bits=cfg.bits, group_size=cfg.group, hadamard=cfg.hadamard)
    same = float((c2.codes == c.codes).float().mean())
    print(f"[full {name}] re-encode byte agreement {same:.5f}", flush=True)
    assert same >= 0.9
    # seeded row sample against the CPU oracle (codes | device L), bit-exact up to ties
    rows = torch.randperm(cfg.rows, generator=torch.Generator().manual_seed(7))[:48].sort().values
    xs = bits16(x[rows.to(dev)])
    lg = bits16(c.L[rows.to(dev)])
    ref = O.encode(xs, bits16(V), cfg.bits, cfg.group, hadamard=cfg.hadamard, l_override=lg)
    assert_codes(c.codes[rows.to(dev)].cpu().numpy(), ref, cfg.bits, what=f"{name} row sample")
    assert np.array_equal(f16(c.scale[rows.to(dev)]).view(np.uint16), ref["scale"].view(np.uint16))


def test_fullsize_fused_equals_decode_then_op(pkg, dev):
    """Config 2 shape: the fused SiLU backward equals decode followed by the dense kernel."""
    cfg = pkg.inputs.CONFIGS["c2"]
    print(f"[full c2] {cfg.rows}x{cfg.hidden}", flush=True)
    x = pkg.inputs.activation(cfg.rows, cfg.hidden, 0, 1.0, cfg.seed, dev)
    V = pkg.inputs.basis(cfg.hidden, cfg.rank, cfg.seed)
    dy = pkg.inputs.gradient((cfg.rows, cfg.hidden), cfg.grad_std, cfg.seed, dev)
    c = pkg.encode(x, V.to(dev), bits=cfg.bits, group_size=cfg.group)
    fused = pkg.silu_backward_compressed(c, dy)
    unfused = pkg.triton_silu_backward(pkg.decode(c), dy)
    torch.cuda.synchronize()
    assert torch.equal(fused, unfused)



def test_fullsize_lora_gradients_on_codes(pkg, dev):
    """lora config (the north-star format at its full size): x_hat^T g from the codes is within
    the fp32 accumulation bound 1e-5 * |x_hat|^T |g| of the float64 product on lrq_decode's
    x_hat (the one dequant_gemm_t is defined on); x_hat A within relative L2 1e-5 and max-abs
    1e-3 of the float64 product (dequant_gemm's x_hat matches lrq_decode's to 1 ulp)."""
    cfg = pkg.inputs.CONFIGS["lora"]
    print(f"[full lora] {cfg.rows}x{cfg.hidden} n={cfg.lora_rank}", flush=True)
    inp = pkg.inputs.make(cfg, device=dev)
    c = pkg.encode(inp["x"], inp["V"].to(dev), bits=cfg.bits, group_size=cfg.group)
    xa = pkg.dequant_gemm(c, inp["a"])
    da = pkg.dequant_gemm_t(c, inp["g"])
    xd = pkg.decode(c).double()
    a, g = inp["a"].double(), inp["g"].double()
    torch.cuda.synchronize()
    ref_da = xd.T @ g
    bound = 1e-5 * (xd.abs().T @ g.abs()) + 1e-12
    worst = float(((da.double() - ref_da).abs() / bound).max())
    print(f"[full lora] dA worst error / bound {worst:.3f}", flush=True)
    assert worst <= 1.0
    ref_xa = xd @ a
    rel = float((xa.double() - ref_xa).norm() / ref_xa.norm())
    mx = float((xa.double() - ref_xa).abs().max())
    print(f"[full lora] xA rel-L2 {rel:.2e} max-abs {mx:.2e}", flush=True)
    assert rel <= 1e-5 and mx <= 1e-3
    # both products from one pass over the codes (lora_grads), fp32 out: each within the fp32
    # accumulation bound of its float64 product
    xa1, da1 = pkg.lora_grads(c, inp["a"], inp["g"], xa_dtype=torch.float32, da_dtype=torch.float32)
    torch.cuda.synchronize()
    w_da = float(((da1.double() - ref_da).abs() / bound).max())
    w_xa = float(((xa1.double() - ref_xa).abs() / (1e-5 * (xd.abs() @ a.abs()) + 1e-12)).max())
    print(f"[full lora] one pass: dA worst error / bound {w_da:.3f}, xA {w_xa:.3f}", flush=True)
    assert w_da <= 1.0 and w_xa <= 1.0


def _prev_bf16(v: float) -> float:
    """The largest bf16 value below the positive bf16 value v."""
    b = torch.tensor(v, dtype=torch.bfloat16).view(torch.int16)
    return (b - 1).view(torch.bfloat16).item()


def test_fullsize_legacy_outliers(pkg, dev):
    """legacy config (the reference's format at [16384, 4096], 2-bit, threshold at 1 %):

      * the GPU threshold tau is the k-th smallest |residual| of the encode's own residual:
        at most numel - k entries exceed tau, more than numel - k reach it (the encode's
        outlier count at tau and at the bf16 value below tau);
      * tau agrees with torch.kthvalue of torch's own bf16 residual to within one bf16 step;
      * the GPU COO compaction equals torch's to_sparse of the same dense outliers, entry for
        entry, and the decode from COO pieces equals the dense decode bit for bit."""
    cfg = pkg.inputs.CONFIGS["legacy"]
    print(f"[full legacy] {cfg.rows}x{cfg.hidden} bits={cfg.bits}", flush=True)
    ops = pkg.inputs.legacy_operands(cfg, dev)
    l, r, s = ops["l"], ops["r"], ops["s"]
    x = pkg.inputs.activation(cfg.rows, cfg.hidden, cfg.n_outlier, cfg.outlier_scale, cfg.seed, dev)[None]
    numel = cfg.rows * cfg.hidden
    k = int(numel * 0.99)
    tau = pkg.outlier_threshold(l, r, x).item()
    assert tau > 0
    oc, q = pkg.legacy_encode_coo(l, r, x, s, quantize_bit=cfg.bits, outlier=tau)
    below, _ = pkg.legacy_encode_coo(l, r, x, s, quantize_bit=cfg.bits, outlier=_prev_bf16(tau))
    n_above, n_reach = int(oc.nnz.item()), int(below.nnz.item())
    print(f"[full legacy] tau {tau} above {n_above} reach {n_reach} numel-k {numel - k}", flush=True)
    assert n_above <= numel - k < n_reach
    oc.check()
    below.check()
    resid = (x[0] - l @ r).abs().flatten().float()
    ref_tau = torch.kthvalue(resid, k).values.item()
    del resid
    assert abs(tau - ref_tau) <= 2.0 ** -7 * ref_tau, (tau, ref_tau)
    o_sp, q2 = pkg.low_rank_addition_fuse_compression_quantization(l, r, x, s, quantize_bit=cfg.bits, outlier=tau)
    assert torch.equal(q, q2)
    dense = o_sp.to_dense()
    ref_sp = dense.to_sparse()
    assert o_sp._nnz() == ref_sp._nnz() == n_above
    assert torch.equal(o_sp.indices(), ref_sp.indices())
    assert torch.equal(o_sp.values().view(torch.int16), ref_sp.values().view(torch.int16))
    xa = pkg.low_rank_addition_fuse_decompression_dequantization(l, r, q, oc, s, quantize_bit=cfg.bits)
    xb = pkg.low_rank_addition_fuse_decompression_dequantization(l, r, q, dense, s, quantize_bit=cfg.bits)
    torch.cuda.synchronize()
    assert torch.equal(xa, xb)


def _row_sample(n_rows: int, k: int = 48, seed: int = 7) -> torch.Tensor:
    return torch.randperm(n_rows, generator=torch.Generator().manual_seed(seed))[:k].sort().values


def test_fullsize_c3_outlier_channels_gelu(pkg, dev):
    """Config 3 at its full [16384, 4096] (the column abs-max over 32 row groups meeting in
    atomics, the top-41 selection, the int8/g128 encode with side columns, the fused GELU
    backward):
      * the column abs-max equals torch's amax of |x| exactly and the top-41 set equals
        torch.topk's (the x50 channels stand clear of the rest);
      * the side columns are fp16(x) of those channels and the decode returns them;
      * every other element is within half a quantisation step of x (channels zeroed);
      * a seeded row sample: codes bit-exact to the oracle (up to ties), the decode equal to the
        oracle's decode of the device codes, the GELU backward within the floating-point bars;
      * the fused GELU backward equals decode followed by the dense GELU kernel on every row."""
    cfg = pkg.inputs.CONFIGS["c3"]
    M, N, k = cfg.rows, cfg.hidden, cfg.keep_channels
    print(f"[full c3] {M}x{N} top-{k}", flush=True)
    x = pkg.inputs.activation(M, N, cfg.n_outlier, cfg.outlier_scale, cfg.seed, dev)
    dy = pkg.inputs.gradient((M, N), cfg.grad_std, cfg.seed, dev)
    cm = pkg.column_absmax(x)
    idx = pkg.topk_channels(cm, k)
    torch.cuda.synchronize()
    cm_ref = x.float().abs().amax(dim=0)
    assert torch.equal(cm, cm_ref)
    top = torch.sort(cm_ref, descending=True).values
    assert float(top[k - 1]) > 5 * float(top[k])
    assert torch.equal(idx.long(), torch.topk(cm_ref, k).indices.sort().values)
    print("[full c3] encode + gelu", flush=True)
    c = pkg.encode(x, None, bits=cfg.bits, group_size=cfg.group, outlier_idx=idx)
    out = pkg.gelu_backward_compressed(c, dy)
    xh = pkg.decode(c)
    torch.cuda.synchronize()
    il = idx.long()
    assert torch.equal(c.side, x[:, il].to(torch.float16))
    assert torch.equal(xh[:, il], c.side.to(torch.bfloat16))
    G = cfg.group
    r = x.float().clone()
    r[:, il] = 0.0
    codes = c.codes.to(torch.int32).float().view(M, -1, G)
    d = codes * c.scale.float()[..., None] + c.zero.float()[..., None]
    err = (d.view(M, -1) - r).abs().view(M, -1, G)
    step = c.scale.float()[..., None]
    bound = 0.5 * step * (1 + 2e-3) + r.abs().view(M, -1, G) * 2e-6 + 1e-6
    frac_ok = float((err <= bound).float().mean())
    print(f"[full c3] within half-step: {frac_ok:.7f}", flush=True)
    assert frac_ok >= 1 - 1e-6
    del r, codes, d, err, bound
    assert torch.equal(out, pkg.triton_gelu_backward(xh, dy))
    rows = _row_sample(M)
    rd = rows.to(dev)
    idx_np = idx.cpu().numpy()
    ref = O.encode(bits16(x[rd]), None, cfg.bits, G, outlier_idx=idx_np)
    assert_codes(c.codes[rd].cpu().numpy(), ref, cfg.bits, what="c3 row sample")
    ref_xh = O.decode(None, None, c.codes[rd].cpu().numpy(), f16(c.scale[rd]), f16(c.zero[rd]), cfg.bits, G,
                      side=f16(c.side[rd]), idx=idx_np)
    assert np.array_equal(bits16(xh[rd]), ref_xh)
    rep = assert_fp_close(bits16(out[rd]), O.gelu_bwd(O.bf16_to_f32(ref_xh), O.bf16_to_f32(bits16(dy[rd]))),
                          "c3 full-size GELU row sample")
    print(f"[full c3] row sample {rep}", flush=True)


def test_fullsize_c5_softmax_rows(pkg, dev):
    """Config 5 at its full 131,072 rows x 2048 (k_softmax_rows walking many row blocks per
    workgroup):
      * on every row, sum_i dS_i = (sum_i dP_i P_i) (1 - sum_i P_i) on the device's own decode P,
        within the bf16 rounding of each dS_i (2^-7 sum |dS_i|) plus the fp32 row sum's
        accumulation (2e-4 sum |dP_i P_i|); a backward missing the row-sum term misses this by
        about sum dP_i P_i;
      * a seeded row sample: the decode against the oracle's decode of the device codes, and dS
        within the floating-point bars of the oracle's decompress-then-op."""
    cfg = pkg.inputs.CONFIGS["c5"]
    M, N = cfg.rows, cfg.hidden
    print(f"[full c5] {M}x{N}", flush=True)
    p = pkg.inputs.softmax_probs((M, N), seed=cfg.seed, device=dev)
    dp = pkg.inputs.gradient((M, N), cfg.grad_std, cfg.seed, dev)
    V = pkg.inputs.basis(N, cfg.rank, cfg.seed)
    c = pkg.encode(p, V.to(dev), bits=cfg.bits, group_size=cfg.group)
    ds = pkg.softmax_backward_compressed(c, dp)
    ph = pkg.decode(c)
    torch.cuda.synchronize()
    worst = 0.0
    for r0 in range(0, M, 16384):  # float64 row sums in slices of 16384 rows
        sl = slice(r0, min(M, r0 + 16384))
        p64, dp64, ds64 = ph[sl].double(), dp[sl].double(), ds[sl].double()
        prod = dp64 * p64
        s = prod.sum(-1)
        psum = p64.sum(-1)
        lhs = ds64.sum(-1)
        rhs = s * (1.0 - psum)
        bound = 2.0 ** -7 * ds64.abs().sum(-1) + 2e-4 * prod.abs().sum(-1) * psum.abs() + 1e-12
        worst = max(worst, float(((lhs - rhs).abs() / bound).max()))
    print(f"[full c5] row-sum identity: worst error / bound {worst:.3f}", flush=True)
    assert worst <= 1.0
    rows = _row_sample(M)
    rd = rows.to(dev)
    ref_ph = O.decode(bits16(c.L[rd]), bits16(V), c.codes[rd].cpu().numpy(), f16(c.scale[rd]), f16(c.zero[rd]),
                      cfg.bits, cfg.group)
    rep_d = assert_decode_close(bits16(ph[rd]), ref_ph, "c5 full-size decode row sample")
    ref = O.softmax_bwd(O.bf16_to_f32(ref_ph), O.bf16_to_f32(bits16(dp[rd])))
    rep = assert_fp_close(bits16(ds[rd]), ref, "c5 full-size softmax row sample", max_abs=1e-3)
    print(f"[full c5] row sample decode {rep_d} dS {rep}", flush=True)


def test_fullsize_decode_xcd_split_equals_halves(pkg, dev):
    """At the north-star shape the plain decode runs its XCD-weighted schedule (pairs of
    workgroups split 32 row blocks as 18 + 14); decoding the same codes as two halves of 8192
    rows (the kernel's loop, no split) gives the same bits, and a row sample from both kinds of
    run matches the CPU oracle's decode."""
    cfg = pkg.inputs.CONFIGS["north_star"]
    M, N = cfg.rows, cfg.hidden
    print(f"[full decode split] {M}x{N}", flush=True)
    x = pkg.inputs.activation(M, N, cfg.n_outlier, cfg.outlier_scale, cfg.seed + 5, dev)
    V = pkg.inputs.basis(N, cfg.rank, cfg.seed)
    c = pkg.encode(x, V.to(dev), bits=cfg.bits, group_size=cfg.group)
    whole = pkg.decode(c)
    halves = []
    for h in range(2):
        sl = slice(h * M // 2, (h + 1) * M // 2)
        part = pkg.CompressedActivation(codes=c.codes[sl], qparams=c.qparams[sl], L=c.L[sl], basis=c.basis,
                                        side=None, idx=None, shape=(M // 2, N), bits=c.bits, group=c.group,
                                        hadamard=False)
        halves.append(pkg.decode(part))
    torch.cuda.synchronize()
    assert torch.equal(whole.view(torch.int16), torch.cat(halves).view(torch.int16))
    # rows of even- and odd-XCD workgroups (each pair of workgroups covers 512 rows: the first
    # 288 are the even one's, the rest the odd one's)
    rows = torch.tensor([0, 287, 288, 511, 512 * 17 + 290, M - 1])
    ref = O.decode(bits16(c.L[rows.to(dev)]), bits16(V), c.codes[rows.to(dev)].cpu().numpy(),
                   f16(c.scale[rows.to(dev)]), f16(c.zero[rows.to(dev)]), cfg.bits, cfg.group)
    assert_decode_close(bits16(whole[rows.to(dev)]), ref, "xcd split rows")
