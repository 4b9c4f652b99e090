"""Host offload of the compressed format.

The reference's offload experiments copy the compressed tensors to the host after the
forward (``o.cpu(), q.cpu()``, offload_forward.py:53-55) and back before the gradient
(offload_backward.py:53-63), synchronously.  Here the copies are asynchronous: pinned host
buffers, a copy stream of their own (default priority), and events, so the transfers overlap
whatever the compute stream does meanwhile.

* ``offload(c)`` starts the device -> host copy of a CompressedActivation and returns a
  ``HostCompressed`` at once; the copy is ordered after the work already queued on the current
  stream (the encode that produced ``c``).
* ``prefetch(h, device)`` starts the host -> device copy and returns a CompressedActivation
  whose tensors the current stream may use right away (the stream waits on the copy's event,
  on the GPU, not on the host).
* ``to_state_dict`` / ``from_state_dict`` fix the wire format: plain tensors
  (codes, qparams, L, side, idx, V) and integer metadata, loadable with safetensors or
  ``torch.load(weights_only=True)``.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

import torch

from .api import CompressedActivation, LowRankBasis

__all__ = ["HostCompressed", "offload", "prefetch", "to_state_dict", "from_state_dict", "WIRE_VERSION"]

WIRE_VERSION = 1
_FIELDS = ("codes", "qparams", "L", "side", "idx")


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

    def wait(self) -> "HostCompressed":
        """Block the host until the device -> host copy has landed."""
        if self.event is not None:
            self.event.synchronize()
        return self

    def nbytes(self) -> int:
        return sum(t.numel() * t.element_size() for t in self.tensors.values())


_copy_streams: dict = {}


def _copy_stream(device: torch.device) -> torch.cuda.Stream:
    key = device.index if device.index is not None else torch.cuda.current_device()
    if key not in _copy_streams:
        with torch.cuda.device(key):
            _copy_streams[key] = torch.cuda.Stream()  # default priority
    return _copy_streams[key]


def _device_tensors(c: CompressedActivation) -> dict:
    return {k: getattr(c, k) for k in _FIELDS if getattr(c, k) is not None}


def offload(c: CompressedActivation, stream: Optional[torch.cuda.Stream] = None) -> HostCompressed:
    """Asynchronous device -> host copy of ``c`` into pinned buffers."""
    dev = c.device
    s = stream if stream is not None else _copy_stream(dev)
    s.wait_stream(torch.cuda.current_stream(dev))  # after the producer of c
    host = {}
    with torch.cuda.stream(s):
        for k, t in _device_tensors(c).items():
            h = torch.empty(t.shape, dtype=t.dtype, pin_memory=True)
            h.copy_(t, non_blocking=True)
            t.record_stream(s)  # the device buffer stays alive until the copy is done
            host[k] = h
        ev = torch.cuda.Event()
        ev.record(s)
    return HostCompressed(host, c.basis, tuple(c.shape), c.bits, c.group, c.hadamard, ev)


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
