"""Host offload on the GPU: an asynchronous device -> host -> device round trip of the
compressed format decodes to the same bits, and the copy holds the data as it was when the
offload was requested (later writes to the device buffers do not reach it)."""

import importlib

import pytest
import torch

pytestmark = pytest.mark.gpu


def test_offload_prefetch_round_trip(pkg, dev):
    OF = importlib.import_module("triton-kernel-test_amd.offload")
    x = pkg.inputs.activation(300, 4096, 8, 20.0, seed=9).to(dev)
    V = pkg.inputs.basis(4096, 16, seed=9).to(dev)
    c = pkg.encode(x, V, bits=4, group_size=64)
    ref = pkg.decode(c)
    h = OF.offload(c)
    h.wait()
    c.codes.zero_()  # the host copy is already taken
    c2 = OF.prefetch(h, dev)
    out = pkg.decode(c2)
    torch.cuda.synchronize()
    assert torch.equal(out, ref)
    assert h.nbytes() == c.nbytes()
    # wire format with a basis, on the device
    c3 = OF.from_state_dict(OF.to_state_dict(h), device=dev)
    assert torch.equal(pkg.decode(c3), ref)
