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
from parity import assert_codes, bits16, f16

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
