"""Host offload of the compressed format.

The reference's offload experiments copy the compressed tensors to the host after the
forward (``o.cpu(), q.cpu()``, offload_forward.py:53-55) and back before the gradient
(offload_backward.py:53-63), synchronously.  Here the copies are asynchronous: pinned host
buffers, a copy stream of their own (default priority), and events, so the transfers overlap
whatever the compute stream does meanwhile.

* ``offload(c)`` starts the device -> host copy of a CompressedActivation and returns a
  ``HostCompressed`` at once; the copy is ordered after the work already queued on the current
  stream (the encode that produced ``c``).  The host buffers come from a ``PinnedPool`` (one per
  process by default) and go back to it with ``HostCompressed.release()``: a training loop that
  offloads the same shapes every step allocates pinned memory in its first step only.
* ``prefetch(h, device)`` starts the host -> device copy and returns a CompressedActivation
  whose tensors the current stream may use right away (the stream waits on the copy's event,
  on the GPU, not on the host).
* ``to_state_dict`` / ``from_state_dict`` fix the wire format: plain tensors
  (codes, qparams, L, side, idx, V) and integer metadata, loadable with safetensors or
  ``torch.load(weights_only=True)``.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Optional

import torch

from .api import CompressedActivation, LowRankBasis

__all__ = ["HostCompressed", "PinnedPool", "default_pool", "offload", "prefetch", "to_state_dict",
           "from_state_dict", "WIRE_VERSION"]

WIRE_VERSION = 1
_FIELDS = ("codes", "qparams", "L", "side", "idx")


class PinnedPool:
    """Pinned host buffers reused across offloads.

    ``take(n)`` hands out a flat uint8 buffer of at least ``n`` bytes: a free buffer of the same
    size class (``n`` rounded up to 64 KiB) whose last copies have completed, else a new pinned
    allocation.  ``give(buf, events)`` returns it together with the events of the copies that
    still read or write it; it is handed out again only once every one of them has completed
    (``Event.query()``), so a buffer is never overwritten under a copy in flight.  At most
    ``max_cached_bytes`` are kept; buffers past that are dropped (freed).  Not thread-safe: use
    one pool per thread that offloads.
    """

    GRAIN = 1 << 16

    def __init__(self, max_cached_bytes: int = 16 << 30, alloc=None):
        self.max_cached_bytes = int(max_cached_bytes)
        self._alloc = alloc if alloc is not None else (
            lambda n: torch.empty(n, dtype=torch.uint8, pin_memory=True))
        self._free: dict = {}  # size class -> [(buffer, [events])]
        self.cached_bytes = 0
        self.allocations = 0   # pinned allocations made (pool misses)

    def _cls(self, n: int) -> int:
        return max(self.GRAIN, (int(n) + self.GRAIN - 1) // self.GRAIN * self.GRAIN)

    def take(self, n: int) -> torch.Tensor:
        cls = self._cls(n)
        lst = self._free.get(cls, [])
        for i, (buf, evs) in enumerate(lst):
            if all(e.query() for e in evs):
                del lst[i]
                self.cached_bytes -= cls
                return buf
        self.allocations += 1
        return self._alloc(cls)

    def give(self, buf: torch.Tensor, events=()) -> None:
        cls = buf.numel()
        if cls != self._cls(cls) or self.cached_bytes + cls > self.max_cached_bytes:
            return  # not one of ours, or over the cap: let it be freed
        self._free.setdefault(cls, []).append((buf, [e for e in events if e is not None]))
        self.cached_bytes += cls

    def clear(self) -> None:
        """Drop every cached buffer (each is freed once no copy uses it any more)."""
        self._free.clear()
        self.cached_bytes = 0


_default_pool: Optional[PinnedPool] = None


def default_pool() -> PinnedPool:
    """The process-wide pool ``offload`` uses when it is given none."""
    global _default_pool
    if _default_pool is None:
        _default_pool = PinnedPool()
    return _default_pool


@dataclass
class HostCompressed:
    """A CompressedActivation in pinned host memory (copy possibly still in flight)."""
    tensors: dict
    basis: Optional[LowRankBasis]
    shape: tuple
    bits: int
    group: int
    hadamard: bool
    event: Optional[torch.cuda.Event] = None
    # pool buffers behind `tensors`, and the events of the copies that read them since (prefetch)
    pool: Optional[PinnedPool] = None
    buffers: list = field(default_factory=list)
    readers: list = field(default_factory=list)

    def wait(self) -> "HostCompressed":
        """Block the host until the device -> host copy has landed."""
        if self.event is not None:
            self.event.synchronize()
        return self

    def nbytes(self) -> int:
        return sum(t.numel() * t.element_size() for t in self.tensors.values())

    def release(self) -> None:
        """Give the host buffers back to the pool.  The tensors must not be used afterwards; the
        buffers are reused only after the offload's copy and every prefetch from them completed."""
        if self.pool is not None:
            for b in self.buffers:
                self.pool.give(b, [self.event, *self.readers])
        self.buffers, self.readers, self.tensors = [], [], {}


_copy_streams: dict = {}


def _copy_stream(device: torch.device) -> torch.cuda.Stream:
    key = device.index if device.index is not None else torch.cuda.current_device()
    if key not in _copy_streams:
        with torch.cuda.device(key):
            _copy_streams[key] = torch.cuda.Stream()  # default priority
    return _copy_streams[key]


def _device_tensors(c: CompressedActivation) -> dict:
    return {k: getattr(c, k) for k in _FIELDS if getattr(c, k) is not None}


def _host_view(buf: torch.Tensor, like: torch.Tensor) -> torch.Tensor:
    n = like.numel() * like.element_size()
    return buf[:n].view(like.dtype).view(like.shape)


def offload(c: CompressedActivation, stream: Optional[torch.cuda.Stream] = None,
            pool: Optional[PinnedPool] = None) -> HostCompressed:
    """Asynchronous device -> host copy of ``c`` into pinned buffers from ``pool`` (the process's
    default pool when None)."""
    dev = c.device
    pool = pool if pool is not None else default_pool()
    s = stream if stream is not None else _copy_stream(dev)
    s.wait_stream(torch.cuda.current_stream(dev))  # after the producer of c
    host, bufs = {}, []
    with torch.cuda.stream(s):
        for k, t in _device_tensors(c).items():
            buf = pool.take(t.numel() * t.element_size())
            bufs.append(buf)
            h = _host_view(buf, t)
            h.copy_(t, non_blocking=True)
            t.record_stream(s)  # the device buffer stays alive until the copy is done
            host[k] = h
        ev = torch.cuda.Event()
        ev.record(s)
    return HostCompressed(host, c.basis, tuple(c.shape), c.bits, c.group, c.hadamard, ev, pool, bufs)


def prefetch(h: HostCompressed, device: torch.device, stream: Optional[torch.cuda.Stream] = None
             ) -> CompressedActivation:
    """Asynchronous host -> device copy; the current stream waits for it on the GPU."""
    device = torch.device(device)
    s = stream if stream is not None else _copy_stream(device)
    if h.event is not None:
        s.wait_event(h.event)  # the host buffers are complete
    dev = {}
    with torch.cuda.stream(s):
        for k, t in h.tensors.items():
            d = torch.empty(t.shape, dtype=t.dtype, device=device)
            d.copy_(t, non_blocking=True)
            dev[k] = d
        ev = torch.cuda.Event()
        ev.record(s)
    h.readers.append(ev)  # the host buffers are not reused before this copy has read them
    cur = torch.cuda.current_stream(device)
    cur.wait_event(ev)
    for d in dev.values():
        d.record_stream(cur)
    return CompressedActivation(codes=dev["codes"], qparams=dev["qparams"], L=dev.get("L"), basis=h.basis,
                                side=dev.get("side"), idx=dev.get("idx"), shape=h.shape, bits=h.bits,
                                group=h.group, hadamard=h.hadamard)


def to_state_dict(c: CompressedActivation | HostCompressed) -> dict:
    """Wire format: the tensors plus integer metadata (no pickled objects)."""
    if isinstance(c, HostCompressed):
        c.wait()
        tensors, basis = dict(c.tensors), c.basis
    else:
        tensors, basis = _device_tensors(c), c.basis
    out = {k: v for k, v in tensors.items()}
    if basis is not None:
        out["V"] = basis.V
    out["meta"] = torch.tensor([WIRE_VERSION, c.bits, c.group, int(c.hadamard), len(c.shape), *c.shape],
                               dtype=torch.int64)
    return out


def from_state_dict(sd: dict, device: Optional[torch.device] = None) -> CompressedActivation:
    """Inverse of ``to_state_dict`` (tensors moved to ``device`` when given)."""
    meta = [int(v) for v in sd["meta"].tolist()]
    if meta[0] != WIRE_VERSION:
        raise ValueError(f"wire format version {meta[0]}, expected {WIRE_VERSION}")
    bits, group, hadamard, nd = meta[1], meta[2], bool(meta[3]), meta[4]
    shape = tuple(meta[5:5 + nd])
    mv = (lambda t: t.to(device)) if device is not None else (lambda t: t)
    basis = None
    if "V" in sd:
        v = mv(sd["V"])
        if not v.is_cuda:
            raise ValueError("an activation of rank > 0 needs a device for its basis")
        basis = LowRankBasis(v)
    get = lambda k: mv(sd[k]) if k in sd else None  # noqa: E731
    return CompressedActivation(codes=get("codes"), qparams=get("qparams"), L=get("L"), basis=basis,
                                side=get("side"), idx=get("idx"), shape=shape, bits=bits, group=group,
                                hadamard=hadamard)
