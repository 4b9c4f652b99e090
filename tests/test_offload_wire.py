"""Wire format of the compressed activation (host offload, CPU): tensors and integer
metadata survive a safetensors round trip unchanged; version mismatches are refused."""

import importlib

import pytest
import torch


def _fake(pkg):
    g = torch.Generator().manual_seed(1)
    rows, n, k = 40, 1024, 3
    return pkg.CompressedActivation(
        codes=torch.randint(0, 256, (rows, n // 2), generator=g, dtype=torch.uint8),
        qparams=torch.randn(rows, n // 128, 2, 2, generator=g).to(torch.float16),
        L=None, basis=None,
        side=torch.randn(rows, k, generator=g).to(torch.float16),
        idx=torch.tensor([3, 70, 900], dtype=torch.int32),
        shape=(2, 20, n), bits=4, group=64, hadamard=False)


def test_wire_round_trip(pkg, tmp_path):
    OF = importlib.import_module("triton-kernel-test_amd.offload")
    c = _fake(pkg)
    sd = OF.to_state_dict(c)
    safetensors = pytest.importorskip("safetensors.torch")
    f = tmp_path / "act.safetensors"
    safetensors.save_file(sd, str(f))
    c2 = OF.from_state_dict(safetensors.load_file(str(f)))
    for k in ("codes", "qparams", "side", "idx"):
        assert torch.equal(getattr(c, k), getattr(c2, k))
    assert (c2.shape, c2.bits, c2.group, c2.hadamard, c2.L) == (c.shape, c.bits, c.group, c.hadamard, None)


def test_wire_version_refused(pkg):
    OF = importlib.import_module("triton-kernel-test_amd.offload")
    sd = OF.to_state_dict(_fake(pkg))
    sd["meta"][0] = OF.WIRE_VERSION + 1
    with pytest.raises(ValueError):
        OF.from_state_dict(sd)
