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


class _Ev:
    """Stands in for a copy's event: complete once `done` is set."""

    def __init__(self, done=False):
        self.done = done

    def query(self):
        return self.done


def test_pinned_pool_reuses_after_the_copies_complete():
    """PinnedPool (CPU, plain buffers in place of pinned ones): a returned buffer is handed out
    again only once every event given with it has completed, within its size class; the cap
    drops buffers instead of caching them."""
    OF = importlib.import_module("triton-kernel-test_amd.offload")
    pool = OF.PinnedPool(max_cached_bytes=3 << 16, alloc=lambda n: torch.empty(n, dtype=torch.uint8))
    a = pool.take(1000)
    assert a.numel() == 1 << 16 and pool.allocations == 1
    pending, done = _Ev(False), _Ev(True)
    pool.give(a, [done, pending])
    b = pool.take(5000)  # same size class, but a copy still uses `a`
    assert b.data_ptr() != a.data_ptr() and pool.allocations == 2
    pending.done = True
    c = pool.take(60000)
    assert c.data_ptr() == a.data_ptr() and pool.allocations == 2
    big = pool.take((1 << 16) + 1)  # the next size class
    assert big.numel() == 2 << 16 and pool.allocations == 3
    pool.give(big, [done])
    pool.give(b, [done])
    assert pool.cached_bytes == 3 << 16
    pool.give(c, [done])  # over the cap: dropped
    assert pool.cached_bytes == 3 << 16
    assert pool.take(10).data_ptr() == b.data_ptr()
    pool.clear()
    assert pool.cached_bytes == 0
