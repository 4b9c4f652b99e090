"""Compress-on-save in autograd (the LoRA layer of the reference's system profiles,
low_rank_system_profile_forward.py:8-18 / low_rank_system_profile_backward.py:55-61, and a
saved-tensor hook for any model).  The forward is unchanged; the gradients are exactly those
of the decoded activation, and close to the uncompressed ones."""

import importlib

import pytest
import torch

pytestmark = pytest.mark.gpu


def _rel(a, b):
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    return float((a - b).norm() / b.norm())


def _f64_lora(x, w, a, b, dy):
    """y and (dx, dA, dB) of y = x W^T + (x A) B by torch autograd in float64 on the CPU: an
    independent evaluation of compute_lora / compute_lora_gradient
    (low_rank_system_profile_forward.py:8-18), with x the activation the gradient sees."""
    d1, d2 = w.shape[1], w.shape[0]
    x64 = x.reshape(-1, d1).double().cpu().requires_grad_()
    a64 = a.double().cpu().requires_grad_()
    b64 = b.double().cpu().requires_grad_()
    y = x64 @ w.double().cpu().T + (x64 @ a64) @ b64
    y.backward(dy.reshape(-1, d2).double().cpu())
    return y.detach(), x64.grad, a64.grad, b64.grad


# bf16 GEMMs with fp32 accumulation round the weight sum and each output once: against the
# float64 gradients the formulas land at ~2.5e-3 relative L2 (measured on the CPU on this
# recipe); a wrong operand (transposed, permuted rows) lands above 0.3
LORA_REL = 5e-3


@pytest.mark.parametrize("fused", [False, True])
def test_lora_linear_compressed(pkg, dev, fused):
    """The LoRA Function's forward and its dx / dA / dB against torch autograd in float64 of
    y = x W^T + (x A) B on the decoded activation; fused=False also equals the formulas on the
    decoded x bit for bit, fused=True (dA and x A from the codes) stays within a few bf16
    roundings of them."""
    AG = importlib.import_module("triton-kernel-test_amd.autograd")
    g = torch.Generator().manual_seed(3)
    d1, d2, r = 1024, 2048, 16
    x = torch.randn(2, 64, d1, generator=g).to(torch.bfloat16).to(dev).requires_grad_()
    w = (torch.randn(d2, d1, generator=g) / d1 ** 0.5).to(torch.bfloat16).to(dev)
    a = (torch.randn(d1, r, generator=g) / d1 ** 0.5).to(torch.bfloat16).to(dev).requires_grad_()
    b = (torch.randn(r, d2, generator=g) * 0.1).to(torch.bfloat16).to(dev).requires_grad_()
    dy = torch.randn(2, 64, d2, generator=g).to(torch.bfloat16).to(dev)
    y = AG.lora_linear_compressed(x, w, a, b, bits=4, group=64, fused=fused)
    y.backward(dy)
    # the gradient sees the decoded activation (the encode is deterministic: same codes)
    xh = pkg.decode(pkg.encode(x.detach(), None, bits=4, group_size=64))
    y0, _, _, _ = _f64_lora(x.detach(), w, a.detach(), b.detach(), dy)
    _, rx, ra, rb = _f64_lora(xh, w, a.detach(), b.detach(), dy)
    rep = {"y": _rel(y.reshape(-1, d2), y0), "dx": _rel(x.grad.reshape(-1, d1), rx), "dA": _rel(a.grad, ra),
           "dB": _rel(b.grad, rb)}
    print(f"[autograd] fused={fused} vs float64 autograd: {rep}", flush=True)
    assert all(v <= LORA_REL for v in rep.values()), rep
    # the comparison catches a wrong factor: dB from the decoded rows in reverse order fails it
    planted = (xh.reshape(-1, d1).flip(0) @ a.detach()).mT @ dy.reshape(-1, d2)
    assert _rel(planted, rb) > 0.1
    dx, da, db = AG.compute_lora_gradient(dy.reshape(-1, d2), xh.reshape(-1, d1), w, a.detach(), b.detach())
    assert torch.equal(x.grad, dx.reshape(x.shape))
    if fused:
        assert _rel(a.grad, da) < 4e-3 and _rel(b.grad, db) < 4e-3
    else:
        assert torch.equal(a.grad, da) and torch.equal(b.grad, db)
    # and close to the uncompressed gradient (int4 / g64 quantisation of x)
    _, _, ra0, rb0 = _f64_lora(x.detach(), w, a.detach(), b.detach(), dy)
    print(f"[autograd] vs uncompressed: dA rel {_rel(a.grad, ra0):.4f} dB rel {_rel(b.grad, rb0):.4f}", flush=True)
    assert _rel(a.grad, ra0) < 0.1 and _rel(b.grad, rb0) < 0.1


def test_saved_tensor_hooks_mlp(pkg, dev):
    AG = importlib.import_module("triton-kernel-test_amd.autograd")
    torch.manual_seed(0)
    mlp = torch.nn.Sequential(torch.nn.Linear(1024, 4096, bias=False), torch.nn.SiLU(),
                              torch.nn.Linear(4096, 1024, bias=False)).to(dev, torch.bfloat16)
    x = torch.randn(256, 1024, device=dev, dtype=torch.bfloat16)

    def grads(hooks):
        mlp.zero_grad(set_to_none=True)
        if hooks is None:
            y = mlp(x)
        else:
            with hooks:
                y = mlp(x)
        y.float().square().sum().backward()
        return [p.grad.clone() for p in mlp.parameters()]

    ref = grads(None)
    hooks = AG.compressed_saved_tensors(bits=8, group=64, min_numel=1)
    got = grads(hooks)
    print(f"[autograd] hook stats {hooks.stats}", flush=True)
    assert hooks.stats["compressed"] >= 2 and hooks.stats["bytes_out"] < hooks.stats["bytes_in"]
    for gg, rr in zip(got, ref):
        assert _rel(gg, rr) < 0.05, _rel(gg, rr)


def test_fit_basis(pkg, dev):
    AG = importlib.import_module("triton-kernel-test_amd.autograd")
    g = torch.Generator().manual_seed(5)
    n, r = 1024, 16
    # rows = a rank-r signal plus noise: the fitted basis captures it
    u = torch.randn(512, r, generator=g)
    vt = torch.linalg.qr(torch.randn(n, r, generator=g)).Q.mT
    x = (u @ vt * 4 + 0.05 * torch.randn(512, n, generator=g)).to(torch.bfloat16).to(dev)
    basis = AG.fit_basis(x, r)
    V = basis.V.float()
    assert float((V.mT @ V - torch.eye(r, device=dev)).abs().max()) < 2e-2
    e0 = (pkg.decode(pkg.encode(x, None, bits=4)).float() - x.float()).norm()
    e1 = (pkg.decode(pkg.encode(x, basis, bits=4)).float() - x.float()).norm()
    print(f"[autograd] round-trip error rank 0 {float(e0):.3f}, fitted rank {r} {float(e1):.3f}", flush=True)
    assert e1 < 0.5 * e0
