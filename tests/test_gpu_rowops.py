"""GPU parity of the row-reducing consumers on the group-mode format: the fused softmax
backward (config 5 recipe, reduced rows) and the fused dequant-GEMM (R12 build shape,
reduced rows).  The reference result is decompress-then-op on the device's own compressed
representation: x_hat = bf16(oracle decode of the device codes), then the formula in
float64, rounded once (tests/parity.py bars).
"""

import numpy as np
import pytest
import torch

import oracle as O
from parity import assert_fp_close, bits16, f16

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


def test_softmax_bwd_unsupported_width(pkg, dev):
    """A row that does not fit one workgroup (32 units) is refused, not computed wrongly."""
    x = torch.rand(16, 4096, dtype=torch.float32).to(torch.bfloat16)
    c = pkg.encode(x.to(dev), None, bits=4, group_size=64)
    with pytest.raises(ValueError):
        pkg.softmax_backward_compressed(c, x.to(dev))


@pytest.mark.parametrize("rows,hidden,rank,n_out,out_dtype", [
    (100, 4096, 16, 32, torch.float32),   # R12 build shape (reduced rows), fp32 out
    (64, 4096, 16, 32, torch.bfloat16),   # bf16 out
    (50, 2048, 0, 16, torch.float32),     # rank 0, n = 16
])
def test_dequant_gemm(pkg, dev, rows, hidden, rank, n_out, out_dtype):
    print(f"[gemm] rows={rows} hidden={hidden} rank={rank} n={n_out} {out_dtype}", flush=True)
    x = pkg.inputs.activation(rows, hidden, 8, 20.0, seed=21)
    V = pkg.inputs.basis(hidden, rank, seed=21) if rank else None
    g = torch.Generator().manual_seed(22)
    a = (torch.randn(hidden, n_out, generator=g) / np.sqrt(hidden)).to(torch.bfloat16)
    c = pkg.encode(x.to(dev), V.to(dev) if V is not None else None, bits=4, group_size=64)
    out = pkg.dequant_gemm(c, a.to(dev), out_dtype=out_dtype)
    torch.cuda.synchronize()
    xh = _xhat(c, V, 4, 64)
    ref = O.gemm(xh, O.bf16_to_f32(bits16(a)))
    if out_dtype == torch.float32:
        got = out.cpu().numpy().astype(np.float64)
        rel = np.linalg.norm(got - ref) / np.linalg.norm(ref)
        assert rel <= 1e-5 and np.abs(got - ref).max() <= 1e-3, (rel, np.abs(got - ref).max())
    else:
        assert_fp_close(bits16(out), ref, "dequant gemm bf16")
