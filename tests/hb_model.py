"""A happens-before model of device memory, streams and events, for CPU tests
of the runtime's ordering.

The runtime's own staging, checkpoint and gradient-offload code runs
unchanged against stand-ins for ``torch.cuda`` and for the library's device
entry points (installed with ``install``):

* ``Device`` is a byte arena on the host.  Device tensors are views into it
  (``DevTensor``), handed out by a model of torch's caching allocator: a
  block freed on a stream is reused only by an allocation on that stream;
  ``record_stream`` makes a freed block wait for an event on each stream it
  was recorded on; a block carries the freeing host thread's clock (the
  allocator's lock orders the free before the reuse).
* Streams, SDMA copies and host threads carry vector clocks.  Enqueuing work
  on a stream joins the issuing host thread's clock into the stream's;
  ``Event.record`` snapshots the stream's clock, ``Stream.wait_event`` joins
  the snapshot into the waiting stream, and a host wait (``synchronize``, a
  ``query`` that returns True) joins it into the host thread.  Nothing
  completes on its own: a host thread knows of completed work only through
  its waits, so orderings that hold only because the device happened to be
  fast are not taken for granted.
* Every kernel, copy and SDMA copy logs the byte ranges it reads and writes.
  Two accesses of overlapping ranges, at least one a write, by different
  agents conflict unless the earlier happens before the later; each conflict
  is recorded in ``Device.races``.

Host memory stays ordinary (pinned tensors are plain host tensors here);
``Device.outstanding_host_copies`` lists copies into or out of host memory
that the calling host thread has not seen complete.
"""

from __future__ import annotations

import contextlib
import itertools
import threading
from types import SimpleNamespace
from typing import List, Optional

import torch

_ALIGN = 512


class VC(dict):
    """Vector clock: agent -> counter."""

    def join(self, other: Optional[dict]) -> "VC":
        for k, v in (other or {}).items():
            if v > self.get(k, 0):
                self[k] = v
        return self

    def copy(self) -> "VC":
        return VC(self)


class DevTensor(torch.Tensor):
    """A tensor living in a ``Device`` arena (its views stay DevTensors)."""

    def record_stream(self, stream) -> None:
        Device.current.record_stream(self, stream)


class FakeStream:
    def __init__(self, dev: "Device", name: str):
        self.dev, self.name = dev, name
        self.vc = VC({name: 0})
        self.cuda_stream = len(dev.streams) + 1
        self.device = torch.device("cuda", 0)
        dev.streams.append(self)

    def enqueue(self) -> VC:
        """A new operation on this stream, issued by the calling host thread:
        after the stream's earlier work and after what the thread has seen
        complete."""
        with self.dev.lock:
            self.vc.join(self.dev.host())
            self.vc[self.name] += 1
            return self.vc.copy()

    def wait_event(self, ev: "FakeEvent") -> None:
        if not self.dev.skip_waits.get(self.name):
            with self.dev.lock:
                self.vc.join(self.dev.host())
                self.vc.join(ev.vc)

    def synchronize(self) -> None:
        self.dev.host().join(self.vc)

    def query(self) -> bool:
        self.synchronize()
        return True

    def __repr__(self):
        return f"<stream {self.name}>"


class FakeEvent:
    def __init__(self, enable_timing: bool = False, blocking: bool = False, interprocess: bool = False):
        self.vc: Optional[VC] = None

    def record(self, stream: Optional[FakeStream] = None) -> None:
        dev = Device.current
        s = stream if stream is not None else dev.current_stream()
        with dev.lock:
            s.vc.join(dev.host())
            self.vc = s.vc.copy()

    def query(self) -> bool:
        Device.current.host().join(self.vc)
        return True

    def synchronize(self) -> None:
        Device.current.host().join(self.vc)

    def elapsed_time(self, other) -> float:
        return 0.0


class Device:
    """The arena, its allocator model, the streams and the access log."""

    current: "Device" = None

    def __init__(self, arena_bytes: int = 64 << 20):
        self.arena = torch.zeros(arena_bytes, dtype=torch.uint8)
        self.base = self.arena.data_ptr()
        self.size = arena_bytes
        self.lock = threading.RLock()
        self.streams: List[FakeStream] = []
        self._local = threading.local()
        self._hosts = {}
        self.top = 0
        self.free_blocks = []       # [stream, offset, nbytes, clock, events]
        self.live = {}              # offset -> [stream, nbytes, recorded streams]
        self.accesses = []          # (lo, hi, agent, vc, write, what)
        self.host_copies = []       # (agent, vc) of copies touching host memory
        self.races = []
        self.skip_waits = {}        # stream name -> True: its waits are dropped (planted mistakes)
        self.skip_dma_waits = False  # True: SDMA completions are not seen (planted mistakes)
        # True: stream copies that read or write host tensors log those host
        # ranges too, so host buffers shared by copies are checked as well
        self.track_host = False
        self._sdma = itertools.count()
        self.default = FakeStream(self, "compute")
        Device.current = self

    # host threads -------------------------------------------------------
    def host(self) -> VC:
        name = getattr(self._local, "name", None) or threading.current_thread().name
        with self.lock:
            return self._hosts.setdefault(name, VC())

    @contextlib.contextmanager
    def as_host(self, name: str):
        """Run the block as host thread ``name`` (its own clock)."""
        old = getattr(self._local, "name", None)
        self._local.name = name
        try:
            yield
        finally:
            self._local.name = old

    def current_stream(self) -> FakeStream:
        return getattr(self._local, "stream", None) or self.default

    @contextlib.contextmanager
    def stream(self, s: Optional[FakeStream]):
        old = getattr(self._local, "stream", None)
        if s is not None:
            self._local.stream = s
        try:
            yield
        finally:
            self._local.stream = old

    def synchronize(self) -> None:
        for s in self.streams:
            s.synchronize()

    # memory -------------------------------------------------------------
    def is_dev(self, t) -> bool:
        return isinstance(t, torch.Tensor) and self.base <= t.data_ptr() < self.base + self.size

    def span(self, t: torch.Tensor):
        lo = t.data_ptr() - self.base
        return lo, lo + t.numel() * t.element_size()

    def alloc(self, shape, dtype) -> DevTensor:
        shape = tuple(shape[0]) if len(shape) == 1 and isinstance(shape[0], (tuple, list, torch.Size)) else shape
        numel = 1
        for d in shape:
            numel *= int(d)
        esize = torch.empty((), dtype=dtype).element_size()
        nbytes = max(_ALIGN, -(-numel * esize // _ALIGN) * _ALIGN)
        s = self.current_stream()
        with self.lock:
            host = self.host()
            for i, b in enumerate(self.free_blocks):
                bs, off, bn, clock, events = b
                if bs is s and bn >= nbytes:
                    del self.free_blocks[i]
                    host.join(clock)          # the allocator's lock: the free came first
                    for ev in events:         # record_stream events, found complete
                        host.join(ev.vc)
                    if bn > nbytes:
                        self.free_blocks.append([bs, off + nbytes, bn - nbytes, clock, events])
                    break
            else:
                off = self.top
                self.top += nbytes
                if self.top > self.size:
                    raise RuntimeError("hb_model: arena exhausted")
            self.live[off] = [s, nbytes, []]
        flat = self.arena[off:off + numel * esize].view(dtype)
        return flat.view(shape).as_subclass(DevTensor)

    def _block(self, t):
        lo = t.data_ptr() - self.base
        for off, blk in self.live.items():
            if off <= lo < off + blk[1]:
                return off, blk
        raise KeyError("hb_model: tensor not in a live block")

    def free(self, t) -> None:
        """The tensor's block goes back to its stream's free list (what the
        caching allocator does when the last reference dies)."""
        with self.lock:
            off, (s, nbytes, recorded) = self._block(t)
            del self.live[off]
            events = []
            for rs in recorded:
                ev = FakeEvent()
                ev.record(rs)
                events.append(ev)
            self.free_blocks.append([s, off, nbytes, self.host().copy(), events])

    def record_stream(self, t, stream) -> None:
        with self.lock:
            _, blk = self._block(t)
            if stream is not blk[0] and stream not in blk[2]:
                blk[2].append(stream)

    # accesses -----------------------------------------------------------
    def _access(self, lo, hi, agent, vc, write, what):
        for a_lo, a_hi, a_agent, a_vc, a_write, a_what in self.accesses:
            if a_hi <= lo or hi <= a_lo or not (write or a_write) or a_agent == agent:
                continue
            if a_vc.get(a_agent, 0) <= vc.get(a_agent, 0):
                continue        # the earlier access happens before this one
            self.races.append(f"{what} ({agent}, {'write' if write else 'read'} [{lo}, {hi})) unordered "
                              f"with {a_what} ({a_agent}, {'write' if a_write else 'read'} [{a_lo}, {a_hi}))")
        self.accesses.append((lo, hi, agent, vc, write, what))

    def op(self, stream: FakeStream, reads=(), writes=(), what: str = "op") -> VC:
        """A kernel or copy on ``stream`` reading and writing tensors (host
        tensors are ignored, but a copy touching host memory is logged as
        outstanding for ``outstanding_host_copies``)."""
        with self.lock:
            vc = stream.enqueue()
            touches_host = False
            for t in reads:
                if self.is_dev(t):
                    self._access(*self.span(t), stream.name, vc, False, what)
                elif isinstance(t, torch.Tensor):
                    touches_host = True
                    if self.track_host:
                        self._access(*self.host_span(t), stream.name, vc, False, what)
            for t in writes:
                if self.is_dev(t):
                    self._access(*self.span(t), stream.name, vc, True, what)
                elif isinstance(t, torch.Tensor):
                    touches_host = True
                    if self.track_host:
                        self._access(*self.host_span(t), stream.name, vc, True, what)
            if touches_host:
                self.host_copies.append((stream.name, vc))
            return vc

    def sdma_copy(self, src, dst, what: str = "sdma copy") -> VC:
        """An SDMA copy of device ``src`` into host ``dst``: an agent of its
        own, ordered after what its issuing host thread has seen complete."""
        with self.lock:
            name = f"sdma{next(self._sdma)}"
            vc = self.host().copy()
            vc[name] = 1
            self._access(*self.span(src), name, vc, False, what)
            self._access(*self.host_span(dst), name, vc, True, what)
            self.host_copies.append((name, vc))
            return vc

    # host accesses (pinned buffers the copies write and the host reads) --
    def host_span(self, t: torch.Tensor):
        """A host tensor's byte range, in a space of its own (offset by the
        arena size so that it never meets device ranges)."""
        lo = t.data_ptr() + (1 << 62)
        return lo, lo + t.numel() * t.element_size()

    def _host_op(self, t, write: bool, what: str) -> None:
        name = getattr(self._local, "name", None) or threading.current_thread().name
        with self.lock:
            h = self.host()
            h[f"host:{name}"] = h.get(f"host:{name}", 0) + 1
            self._access(*self.host_span(t), f"host:{name}", h.copy(), write, what)

    def host_read(self, t: torch.Tensor, what: str = "host read") -> None:
        self._host_op(t, False, what)

    def host_write(self, t: torch.Tensor, what: str = "host write") -> None:
        self._host_op(t, True, what)

    def outstanding_host_copies(self) -> list:
        h = self.host()
        return [(a, vc) for a, vc in self.host_copies if h.get(a, 0) < vc[a]]


class _Timer:
    def elapsed_ms(self) -> float:
        return 0.0


def fake_kernels(dev: Device):
    """Stand-ins for the ``kernels`` entry points the runtime's ordering code
    calls, logging their accesses."""

    def memcpy_async(dst, src, stream=None, nbytes=None):
        s = stream or dev.current_stream()
        if nbytes is not None and nbytes != dst.numel() * dst.element_size():
            dst = dst.reshape(-1).view(torch.uint8)[:nbytes]
        dev.op(s, reads=[src], writes=[dst], what=f"copy on {s.name}")

    def cast_f32_16_(dst, src, stream=None, timer=None):
        s = stream or dev.current_stream()
        dev.op(s, reads=[src], writes=[dst], what=f"cast on {s.name}")
        return dst

    def copy_segs_b16(pairs, stream=None, max_workgroups=0):
        s = stream or dev.current_stream()
        dev.op(s, reads=[a for a, _ in pairs], writes=[b for _, b in pairs], what=f"pack on {s.name}")

    class DmaReady:
        def __init__(self, handle, timeout=None):
            self.handle = handle
            self.released = False

        def query(self) -> bool:
            if dev.skip_dma_waits:
                return True
            for vc in self.handle:
                dev.host().join(vc)
            return True

        def synchronize(self) -> None:
            self.query()

        def release(self):
            if self.released:
                raise RuntimeError("DmaReady: released twice")
            self.query()
            self.released = True
            return (0, 0)

    def dma_copy_d2h(pairs, timeout=None):
        return [dev.sdma_copy(src, dst, what="SDMA copy") for src, dst in pairs]

    def wait_event(ev, timeout, what):
        ev.synchronize()

    return SimpleNamespace(memcpy_async=memcpy_async, cast_f32_16_=cast_f32_16_, copy_segs_b16=copy_segs_b16,
                           KernelTimer=_Timer, DmaReady=DmaReady, dma_copy_d2h=dma_copy_d2h,
                           wait_event=wait_event, DmaCopiesOutstanding=TimeoutError)


class _FakeCuda:
    def __init__(self, dev: Device):
        self._dev = dev
        self.Event = FakeEvent
        self.OutOfMemoryError = torch.cuda.OutOfMemoryError

    def Stream(self, device=None, priority=0):
        return FakeStream(self._dev, f"stream{len(self._dev.streams)}")

    def stream(self, s):
        return self._dev.stream(s)

    def current_stream(self, device=None):
        return self._dev.current_stream()

    def synchronize(self, device=None):
        self._dev.synchronize()

    def __getattr__(self, name):
        return getattr(torch.cuda, name)


class FakeTorch:
    """``torch`` with device allocations and ``torch.cuda`` redirected."""

    def __init__(self, dev: Device):
        self._dev = dev
        self.cuda = _FakeCuda(dev)

    def empty(self, *size, dtype=None, device=None, **kw):
        if device is not None and "cuda" in str(device):
            return self._dev.alloc(size, dtype or torch.float32)
        return torch.empty(*size, dtype=dtype, **kw)

    def __getattr__(self, name):
        return getattr(torch, name)


def install(monkeypatch, dev: Device, *modules) -> None:
    """Point each module's ``torch`` and ``kernels`` at the model."""
    ft, fk = FakeTorch(dev), fake_kernels(dev)
    for m in modules:
        if hasattr(m, "torch"):
            monkeypatch.setattr(m, "torch", ft)
        if hasattr(m, "kernels"):
            monkeypatch.setattr(m, "kernels", fk)
