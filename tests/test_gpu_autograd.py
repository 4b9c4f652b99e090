"""Compress-on-save in autograd (the LoRA layer of the reference's system profiles,
low_rank_system_profile_forward.py:8-18 / low_rank_system_profile_backward.py:55-61, and a
saved-tensor hook for any model).  The forward is unchanged; the gradients are exactly those
of the decoded activation, and close to the uncompressed ones."""

import importlib

import pytest
import torch

pytestmark = pytest.mark.gpu


def _rel(a, b):
    return float((a.float() - b.float()).norm() / b.float().norm())


@pytest.mark.parametrize("fused", [False, True])
def test_lora_linear_compressed(pkg, dev, fused):
    """fused=False: the formulas on the decoded x, bit for bit.  fused=True: dA and x A read the
    codes (transposed dequant-GEMM / dequant-GEMM, fp32 accumulate, one rounding): within a
    few bf16 roundings of the same formulas."""
    AG = importlib.import_module("triton-kernel-test_amd.autograd")
    g = torch.Generator().manual_seed(3)
    d1, d2, r = 1024, 2048, 16
    x = torch.randn(2, 64, d1, generator=g).to(torch.bfloat16).to(dev).requires_grad_()
    w = (torch.randn(d2, d1, generator=g) / d1 ** 0.5).to(torch.bfloat16).to(dev)
    a = (torch.randn(d1, r, generator=g) / d1 ** 0.5).to(torch.bfloat16).to(dev).requires_grad_()
    b = (torch.randn(r, d2, generator=g) * 0.1).to(torch.bfloat16).to(dev).requires_grad_()
    dy = torch.randn(2, 64, d2, generator=g).to(torch.bfloat16).to(dev)
    y = AG.lora_linear_compressed(x, w, a, b, bits=4, group=64, fused=fused)
    assert torch.equal(y, AG.compute_lora(x.detach(), w, a.detach(), b.detach()))
    y.backward(dy)
    # exactly the gradient formulas on the decoded activation
    xh = pkg.decode(pkg.encode(x.detach(), None, bits=4, group_size=64))
    dx, da, db = AG.compute_lora_gradient(dy.reshape(-1, d2), xh.reshape(-1, d1), w, a.detach(), b.detach())
    assert torch.equal(x.grad, dx.reshape(x.shape))
    if fused:
        print(f"[autograd] fused vs decoded: dA rel {_rel(a.grad, da):.2e} dB rel {_rel(b.grad, db):.2e}",
              flush=True)
        assert _rel(a.grad, da) < 4e-3 and _rel(b.grad, db) < 4e-3
    else:
        assert torch.equal(a.grad, da) and torch.equal(b.grad, db)
    # and close to the uncompressed gradient (int4 / g64 quantisation of x)
    _, da0, db0 = AG.compute_lora_gradient(dy.reshape(-1, d2), x.detach().reshape(-1, d1), w, a.detach(),
                                           b.detach())
    print(f"[autograd] dA rel {_rel(a.grad, da0):.4f} dB rel {_rel(b.grad, db0):.4f}", flush=True)
    assert _rel(a.grad, da0) < 0.1 and _rel(b.grad, db0) < 0.1


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
