"""Device buffers and the per-unit runtime of the layer-streaming path.

Reference layer_state.py:28-467.  The reference casts each unit's fp32
master to bf16 on the host (one thread, layer_state.py:301), copies the bf16
layer to the GPU and blocks on the copy stream (:326); gradients come back
through one shared pinned buffer (:367-381), which serialises each offload
behind the previous unit's CPU update (:362-363).

Here the GPU does the staging, and work on the GPU is ordered with events
instead of host waits:

* Units live in a 2-unit pool (``LayerBufferPool``, the reference's) or in a
  device buffer of their own (``make_resident``): an own buffer keeps the
  forward's weights for the backward, and is staged with the next step's
  weights by the update thread right after the unit's update
  (``stage_for_next_forward``), i.e. during the backward.
* H2D: ``H2DStager`` copies the pinned fp32 master by DMA into a device fp32
  ring on ``h2d_stream`` and a HIP kernel casts it to bf16 (RNE) into the
  unit on ``cast_stream``; with bf16 H2D, ``BF16Loader`` copies the host
  optimizer's bf16 copy straight into the unit.  Either waits for the unit's
  ``ready`` event, after which its previous contents are no longer read (the
  reference has no such fence: layer_state.py:292-315 start the next H2D
  into a unit released on the host without waiting for the compute stream).
* Gradients: once a unit's last gradient is accumulated, the offload thread
  copies the per-parameter bf16 grads straight into a pinned host slot (one
  per unit, ``GradSlotsPerUnit``, or a ring when the host cannot pin that
  much), on SDMA engines or by a capped pack kernel, and queues the update;
  the update thread (``PriorityUpdateExecutor``) runs LayerAdam on the slot,
  taking among the units whose copies have landed the one the next forward
  needs first.
* The embedding unit can be row-sparse (``enable_row_sparse``): only the
  batch's rows are read from the host table and only their gradient rows
  come back.

Memory layout in HBM (per unit, offset-identical to the fp32 master):
  unit["param"]  bf16 weights (pool units: ``max_param_size`` elements)
plus the fp32 staging ring (``depth`` chunks of ``chunk_elems``) with fp32 H2D.
"""

from __future__ import annotations

import bisect
import itertools
import queue
import threading
import time
from collections import OrderedDict, deque
from concurrent.futures import Future
from typing import Any, Callable, Dict, List, Optional, Sequence, Tuple

import torch
import torch.nn as nn

from . import _native, kernels
from .optimizer import cpu_adam as _cpu_adam
from .pinned import pinned_empty


def _new_event() -> torch.cuda.Event:
    return torch.cuda.Event(enable_timing=False, blocking=False)


# Queue priority of work that may wait until the host AdamW has nothing else
# ready (the gradient-free rows of the embedding's update).
EARLY_UPDATE_PRIORITY = 1 << 30


class LayerBufferPool:
    """Fixed set of device units ``{"param", "grad"}`` reused round-robin.

    Reference layer_state.py:28-101 (``acquire`` = popleft, ``release`` =
    append).  Two differences: ``acquire`` blocks until a unit is released
    (units come back from the gradient-offload thread, not only from the
    thread that acquires), and every unit carries a ``ready`` event that the
    next writer of the unit must wait on.
    """

    def __init__(self, max_param_size: int, dtype: torch.dtype, device: torch.device, pool_size: int = 2):
        if pool_size < 2:
            raise ValueError("gpu_buffer_pool_size must be at least 2 (current + prefetched unit)")
        self.max_param_size = max_param_size
        self.dtype = dtype
        self.device = device
        self.pool_size = pool_size
        self.pool: deque = deque()
        for _ in range(pool_size):
            self.pool.append({
                "param": torch.empty(max_param_size, dtype=dtype, device=device),
                "grad": torch.empty(max_param_size, dtype=dtype, device=device),
                "ready": None,
            })
        self._cv = threading.Condition()

    def acquire(self, timeout: Optional[float] = None) -> Dict[str, Any]:
        with self._cv:
            if not self._cv.wait_for(lambda: len(self.pool) > 0, timeout=timeout):
                raise TimeoutError("LayerBufferPool.acquire: no unit released in time")
            return self.pool.popleft()

    def release(self, unit: Dict[str, Any]) -> None:
        with self._cv:
            self.pool.append(unit)
            self._cv.notify()

    def available(self) -> int:
        with self._cv:
            return len(self.pool)


_BACKLOG_LOCK = threading.Lock()


def _backlog(copies: deque) -> int:
    """Drop the completed events at the front of ``copies`` (one stream, so
    they complete in order) and count the rest.  Several threads trim (the
    update thread, the threads that issue copies); appends need no lock."""
    with _BACKLOG_LOCK:
        while copies and copies[0].query():
            copies.popleft()
        return len(copies)


def split_into_pieces(sizes: Sequence[int], piece_elems: int) -> List[Tuple[int, int]]:
    """Flat ``[a, b)`` ranges of about ``piece_elems`` elements covering
    tensors of ``sizes`` laid out back to back.  A boundary inside a tensor
    falls a multiple of 16 elements after that tensor's start, so a host
    AdamW call per piece gives every element the arithmetic of the
    whole-tensor call (16-wide vector body, scalar tail at the end)."""
    total = int(sum(sizes))
    if total == 0:
        return []
    n = max(1, -(-total // int(piece_elems))) if piece_elems and piece_elems > 0 else 1
    starts = list(itertools.accumulate([0] + [int(s) for s in sizes[:-1]]))
    bounds = [0]
    for k in range(1, n):
        c = total * k // n
        i = bisect.bisect_right(starts, c) - 1
        c = starts[i] + (c - starts[i]) // 16 * 16
        if c > bounds[-1]:
            bounds.append(c)
    bounds.append(total)
    return list(zip(bounds[:-1], bounds[1:]))


def overlap_ranges(spans: Sequence[Tuple[int, int]], a: int, b: int) -> List[Tuple[int, int, int]]:
    """``(index, lo, hi)`` for each span ``(offset, size)`` that overlaps the
    flat range ``[a, b)``; ``lo``/``hi`` are relative to the span's offset."""
    out = []
    for i, (off, size) in enumerate(spans):
        lo, hi = max(a, off) - off, min(b, off + size) - off
        if hi > lo:
            out.append((i, lo, hi))
    return out


class _StageTicket:
    """Chunks of one unit's master in flight through the staging ring."""

    def __init__(self, host: torch.Tensor, chunks: List[Tuple[int, int]]):
        self.host = host
        self.chunks = chunks          # (offset, elements) per chunk
        self.slots: List[int] = []    # staging slot of each issued copy
        self.copied: List[torch.cuda.Event] = []


class PendingCast:
    """A unit's fp32 weights copied into a device slot, not yet cast: the
    cast runs where the unit is next used (``H2DStager.cast_pending``)."""

    __slots__ = ("slot", "copied", "n", "wait_event")

    def __init__(self, slot: torch.Tensor, copied: torch.cuda.Event, n: int,
                 wait_event: Optional[torch.cuda.Event]):
        self.slot, self.copied, self.n, self.wait_event = slot, copied, n, wait_event


class _SlotPool:
    """Device fp32 buffers of whole units, keyed by size and reused.  A
    buffer comes back with the event after which it may be overwritten.
    Allocation stops at ``cap_bytes`` or at the first out-of-memory error;
    callers then stage through the ring."""

    def __init__(self, device: torch.device, cap_bytes: int):
        self.device = device
        self.cap_bytes = int(cap_bytes)
        self.bytes = 0
        self.disabled = False
        self._free: Dict[int, List[Tuple[torch.Tensor, Optional[torch.cuda.Event]]]] = {}
        self._lock = threading.Lock()

    def take(self, n: int) -> Optional[Tuple[torch.Tensor, Optional[torch.cuda.Event]]]:
        """A buffer of ``n`` elements: the free one given back last, else a
        new one.  The last one's cast is usually still queued on the forward's
        stream, so the next copy into it waits for the forward to reach that
        cast; measured on one box, 30 steps each, this ran at 5,543 and 5,611
        tokens/s, preferring buffers whose cast had finished (then the oldest)
        at 4,883 and 4,236, and casting as soon as the copy lands at 5,303 and
        5,323."""
        with self._lock:
            free = self._free.get(n)
            if free:
                return free.pop()
            if self.disabled or self.bytes + 4 * n > self.cap_bytes:
                return None
            try:
                t = torch.empty(n, dtype=torch.float32, device=self.device)
            except torch.cuda.OutOfMemoryError:
                self.disabled = True
                return None
            self.bytes += 4 * n
            return t, None

    def give(self, t: torch.Tensor, free_event: Optional[torch.cuda.Event]) -> None:
        with self._lock:
            self._free.setdefault(t.numel(), []).append((t, free_event))

    def release(self) -> None:
        """Drop the free buffers (the caller has made sure nothing still copies
        into or reads from them); buffers still out stay with their holders."""
        with self._lock:
            for lst in self._free.values():
                self.bytes -= sum(4 * t.numel() for t, _ in lst)
            self._free.clear()


class H2DStager:
    """Pinned fp32 master -> device bf16 unit, through a device fp32 ring.

    Two phases, so the host link never waits for a pool unit:
      ``begin``   issues the DMA copies of the first ``depth`` chunks into
                  free ring slots on ``h2d_stream`` (each after the cast that
                  last read its slot) -- no pool unit is needed for this;
      ``finish``  once the caller holds a unit, casts each chunk into it on
                  ``cast_stream`` (after the unit's ``ready`` event and the
                  chunk's copy) and issues the remaining copies as slots free.
    One unit is staged at a time: ``begin`` takes a lock that ``finish``
    releases.

    Units staged right after their update (``copy_for_later``, ``open_pieces``)
    instead land whole in a device fp32 slot of their own size, and their cast
    can wait until the unit is next used (``cast_pending``, on the stream that
    uses it): the cast then runs between that stream's kernels, with the HBM
    to itself, instead of beside the backward's GEMMs.
    """

    def __init__(self, device: torch.device, chunk_elems: int, depth: int,
                 h2d_stream: torch.cuda.Stream, cast_stream: torch.cuda.Stream,
                 slot_cap_bytes: int = 0):
        if depth < 1 or chunk_elems < 1:
            raise ValueError("H2DStager: depth and chunk_elems must be positive")
        self.chunk = int(chunk_elems)
        self.depth = int(depth)
        self.buf = torch.empty(self.depth * self.chunk, dtype=torch.float32, device=device)
        self.slot_free: List[Optional[torch.cuda.Event]] = [None] * self.depth
        self.next_slot = 0
        self.h2d_stream = h2d_stream
        self.cast_stream = cast_stream
        self._lock = threading.Lock()
        # Optional instrumentation: when a list, each cast appends
        # (KernelTimer, None, n_elements), timed around the cast kernels
        # themselves; each copy appends (start_event, end_event, bytes) to
        # copy_timing.
        self.cast_timing: Optional[list] = None
        self.copy_timing: Optional[list] = None
        # Completion event of the last cast issued (see fence_after_casts).
        self.last_cast_done: Optional[torch.cuda.Event] = None
        self._copies: deque = deque()   # completion events of issued copies, in stream order
        # Whole-unit device slots of ``copy_for_later`` and ``open_pieces``.
        self.slots = _SlotPool(device, slot_cap_bytes)

    def backlog(self) -> int:
        """Host-to-device copies issued and not yet complete."""
        return _backlog(self._copies)

    def fence_after_casts(self, stream: torch.cuda.Stream) -> None:
        """Make ``stream`` wait for every cast issued so far.  Kernels that write
        into host memory are ordered behind the casts this way: a PCIe-writing
        kernel running beside the HBM-bound cast slows it severalfold, even on
        disjoint CUs, while delaying the writer by one cast costs nothing."""
        ev = self.last_cast_done
        if ev is not None:
            stream.wait_event(ev)

    def _slot(self, s: int, c: int) -> torch.Tensor:
        return self.buf[s * self.chunk: s * self.chunk + c]

    def _issue_copy(self, t: _StageTicket, j: int) -> None:
        off, c = t.chunks[j]
        s = self.next_slot
        self.next_slot = (s + 1) % self.depth
        if self.slot_free[s] is not None:
            self.h2d_stream.wait_event(self.slot_free[s])
        timing = self.copy_timing is not None
        if timing:
            t0 = torch.cuda.Event(enable_timing=True)
            t0.record(self.h2d_stream)
        kernels.memcpy_async(self._slot(s, c), t.host[off:off + c], self.h2d_stream)
        copied = torch.cuda.Event(enable_timing=True) if timing else _new_event()
        copied.record(self.h2d_stream)
        if timing:
            self.copy_timing.append((t0, copied, c * 4))
        t.slots.append(s)
        t.copied.append(copied)
        self._copies.append(copied)
        if len(self._copies) > 64:
            _backlog(self._copies)

    def begin(self, host_f32: torch.Tensor) -> _StageTicket:
        self._lock.acquire()
        try:
            n = host_f32.numel()
            t = _StageTicket(host_f32, [(off, min(self.chunk, n - off)) for off in range(0, n, self.chunk)])
            for j in range(min(len(t.chunks), self.depth)):
                self._issue_copy(t, j)
            return t
        except BaseException:
            self._lock.release()
            raise

    def finish(self, t: _StageTicket, dst_bf16: torch.Tensor,
               wait_event: Optional[torch.cuda.Event]) -> torch.cuda.Event:
        try:
            if dst_bf16.numel() < t.host.numel():
                raise ValueError("H2DStager.finish: destination smaller than source")
            if wait_event is not None:
                self.cast_stream.wait_event(wait_event)
            timing = self.cast_timing is not None
            for j, (off, c) in enumerate(t.chunks):
                s = t.slots[j]
                self.cast_stream.wait_event(t.copied[j])
                timer = kernels.KernelTimer() if timing else None
                kernels.cast_f32_bf16_(dst_bf16[off:off + c], self._slot(s, c), self.cast_stream, timer=timer)
                freed = _new_event()
                freed.record(self.cast_stream)
                if timing:
                    self.cast_timing.append((timer, None, c))
                self.slot_free[s] = freed
                if j + self.depth < len(t.chunks):
                    self._issue_copy(t, j + self.depth)  # reuses slot s, after this cast
            done = _new_event()
            done.record(self.cast_stream)
            self.last_cast_done = done
            return done
        finally:
            self._lock.release()

    def load(self, host_f32: torch.Tensor, dst_bf16: torch.Tensor,
             wait_event: Optional[torch.cuda.Event]) -> torch.cuda.Event:
        """``begin`` and ``finish`` in one call."""
        return self.finish(self.begin(host_f32), dst_bf16, wait_event)

    def copy_for_later(self, host_f32: torch.Tensor,
                       wait_event: Optional[torch.cuda.Event]) -> Optional[PendingCast]:
        """Copy the whole unit into a device slot of its size on ``h2d_stream``
        (after that slot's last cast); the cast is left to ``cast_pending``.
        ``wait_event`` is what the cast must wait for besides the copy (the
        destination's last reader).  None when no slot can be had."""
        n = host_f32.numel()
        got = self.slots.take(n)
        if got is None:
            return None
        slot, free_ev = got
        if free_ev is not None:
            self.h2d_stream.wait_event(free_ev)
        timing = self.copy_timing is not None
        if timing:
            t0 = torch.cuda.Event(enable_timing=True)
            t0.record(self.h2d_stream)
        kernels.memcpy_async(slot[:n], host_f32, self.h2d_stream)
        copied = torch.cuda.Event(enable_timing=True) if timing else _new_event()
        copied.record(self.h2d_stream)
        if timing:
            self.copy_timing.append((t0, copied, n * 4))
        self._copies.append(copied)
        if len(self._copies) > 64:
            _backlog(self._copies)
        return PendingCast(slot, copied, n, wait_event)

    def cast_pending(self, p: PendingCast, dst_bf16: torch.Tensor, stream: torch.cuda.Stream) -> torch.cuda.Event:
        """Cast a copied unit into ``dst_bf16`` on ``stream`` (after its copy and
        its ``wait_event``); the slot goes back to the pool behind the cast."""
        if dst_bf16.numel() < p.n:
            raise ValueError("H2DStager.cast_pending: destination smaller than the unit")
        if p.wait_event is not None:
            stream.wait_event(p.wait_event)
        stream.wait_event(p.copied)
        timer = kernels.KernelTimer() if self.cast_timing is not None else None
        kernels.cast_f32_bf16_(dst_bf16[:p.n], p.slot[:p.n], stream, timer=timer)
        freed = _new_event()
        freed.record(stream)
        if timer is not None:
            self.cast_timing.append((timer, None, p.n))
        self.slots.give(p.slot, freed)
        self.last_cast_done = freed
        return freed

    def drop_pending(self, p: PendingCast) -> None:
        """Give a copied unit's slot back without casting it."""
        self.slots.give(p.slot, p.copied)

    def open_pieces(self, host_f32: torch.Tensor, dst_bf16: torch.Tensor, wait_event: Optional[torch.cuda.Event],
                    pieces: Sequence[Tuple[int, int]]) -> Optional["_StagerPieces"]:
        """Copy ``host_f32`` to the device one flat piece ``[a, b)`` at a time,
        each when the caller ``push``-es it (after writing it), so the copy of
        the first pieces runs while later ones are still being produced.  The
        pieces land in a device slot of the unit's size; ``close`` casts the
        unit into ``dst_bf16`` or leaves the cast to ``cast_pending``.  None
        when no slot can be had."""
        got = self.slots.take(host_f32.numel())
        if got is None:
            return None
        try:
            return _StagerPieces(self, host_f32, dst_bf16, wait_event, pieces, got)
        except BaseException:
            self.slots.give(*got)
            raise


class _StagerPieces:
    """One unit's copy, piece by piece, into a whole-unit slot of an ``H2DStager``."""

    def __init__(self, stager: H2DStager, host: torch.Tensor, dst: torch.Tensor,
                 wait_event: Optional[torch.cuda.Event], pieces: Sequence[Tuple[int, int]],
                 slot: Tuple[torch.Tensor, Optional[torch.cuda.Event]]):
        n = host.numel()
        if dst.numel() < n:
            raise ValueError("H2DStager.open_pieces: destination smaller than source")
        bounds = [0] + [b for _, b in pieces]
        if not pieces or any(pieces[i][0] != bounds[i] or pieces[i][1] <= pieces[i][0]
                             for i in range(len(pieces))) or bounds[-1] != n:
            raise ValueError("H2DStager.open_pieces: the pieces must cover the source in order")
        self.stager, self.host, self.dst, self.wait_event = stager, host, dst, wait_event
        self.pieces = list(pieces)
        self.buf, self.slot_free = slot
        self.pushed = 0
        self.last_copy: Optional[torch.cuda.Event] = None
        self.open = True

    def push(self, j: int) -> None:
        if not self.open or j != self.pushed:
            raise RuntimeError(f"H2DStager pieces: piece {j} pushed out of order (next is {self.pushed})")
        st = self.stager
        a, b = self.pieces[j]
        if j == 0 and self.slot_free is not None:
            st.h2d_stream.wait_event(self.slot_free)   # the slot's last cast has read it
        timing = st.copy_timing is not None
        if timing:
            t0 = torch.cuda.Event(enable_timing=True)
            t0.record(st.h2d_stream)
        kernels.memcpy_async(self.buf[a:b], self.host[a:b], st.h2d_stream)
        copied = torch.cuda.Event(enable_timing=True) if timing else _new_event()
        copied.record(st.h2d_stream)
        if timing:
            st.copy_timing.append((t0, copied, (b - a) * 4))
        self.pushed += 1
        if self.pushed == len(self.pieces):
            self.last_copy = copied
            # the backlog counts units: queued until the unit's last copy is done
            st._copies.append(copied)
            if len(st._copies) > 64:
                _backlog(st._copies)

    def close(self, cast_later: bool = False):
        """After the last piece: a ``PendingCast`` (``cast_later``) or the
        completion event of the unit's cast on the stager's cast stream."""
        if not self.open or self.pushed != len(self.pieces):
            raise RuntimeError(f"H2DStager pieces: {self.pushed} of {len(self.pieces)} pieces pushed")
        self.open = False
        p = PendingCast(self.buf, self.last_copy, self.host.numel(), self.wait_event)
        if cast_later:
            return p
        return self.stager.cast_pending(p, self.dst, self.stager.cast_stream)

    def abort(self) -> None:
        """Give the slot back without casting (the unit is staged whole later);
        copies already issued finish into it ahead of its next user's copies
        on the same stream."""
        if self.open:
            self.open = False
            self.stager.slots.give(self.buf, None)


class BF16Loader:
    """Pinned bf16 host copy -> device bf16 unit: one DMA per unit, no cast.

    Used when the host optimizer keeps a bf16 copy of every master current
    (it writes it in the same pass as the update), so two bytes per parameter
    cross the host link -- the reference's link format (layer_state.py:299-314)
    without its host cast on the load path.  Offers the stager's fence
    interface; there are no casts to fence behind.
    """

    def __init__(self, h2d_stream: torch.cuda.Stream):
        self.h2d_stream = h2d_stream
        self._copies: deque = deque()
        self.last_cast_done: Optional[torch.cuda.Event] = None
        self.cast_timing: Optional[list] = None
        self.copy_timing: Optional[list] = None

    def fence_after_casts(self, stream: torch.cuda.Stream) -> None:
        return None

    def load(self, host_bf16: torch.Tensor, dst_bf16: torch.Tensor,
             wait_event: Optional[torch.cuda.Event]) -> torch.cuda.Event:
        n = host_bf16.numel()
        if dst_bf16.numel() < n:
            raise ValueError("BF16Loader.load: destination smaller than source")
        if wait_event is not None:
            self.h2d_stream.wait_event(wait_event)
        timing = self.copy_timing is not None
        if timing:
            t0 = torch.cuda.Event(enable_timing=True)
            t0.record(self.h2d_stream)
        kernels.memcpy_async(dst_bf16[:n], host_bf16, self.h2d_stream)
        done = torch.cuda.Event(enable_timing=True) if timing else _new_event()
        done.record(self.h2d_stream)
        if timing:
            self.copy_timing.append((t0, done, n * 2))
        self._copies.append(done)
        if len(self._copies) > 64:
            _backlog(self._copies)
        return done

    def backlog(self) -> int:
        """Host-to-device copies issued and not yet complete."""
        return _backlog(self._copies)

    def open_pieces(self, host_bf16: torch.Tensor, dst_bf16: torch.Tensor, wait_event: Optional[torch.cuda.Event],
                    pieces: Sequence[Tuple[int, int]]) -> "_LoaderPieces":
        """``load`` one flat piece ``[a, b)`` at a time, each when pushed."""
        return _LoaderPieces(self, host_bf16, dst_bf16, wait_event, pieces)


class _LoaderPieces:
    """One unit loaded piece by piece by a ``BF16Loader``."""

    def __init__(self, loader: BF16Loader, host: torch.Tensor, dst: torch.Tensor,
                 wait_event: Optional[torch.cuda.Event], pieces: Sequence[Tuple[int, int]]):
        if dst.numel() < host.numel():
            raise ValueError("BF16Loader.open_pieces: destination smaller than source")
        if any(b <= a for a, b in pieces) or (pieces and pieces[-1][1] > host.numel()):
            raise ValueError("BF16Loader.open_pieces: a piece is empty or outside the source")
        self.loader, self.host, self.dst, self.wait_event = loader, host, dst, wait_event
        self.pieces = list(pieces)
        self.pushed = 0
        self.done: Optional[torch.cuda.Event] = None

    def push(self, j: int) -> None:
        if j != self.pushed:
            raise RuntimeError(f"BF16Loader pieces: piece {j} pushed out of order (next is {self.pushed})")
        ld = self.loader
        a, b = self.pieces[j]
        if j == 0 and self.wait_event is not None:
            ld.h2d_stream.wait_event(self.wait_event)
        timing = ld.copy_timing is not None
        if timing:
            t0 = torch.cuda.Event(enable_timing=True)
            t0.record(ld.h2d_stream)
        kernels.memcpy_async(self.dst[a:b], self.host[a:b], ld.h2d_stream)
        ev = torch.cuda.Event(enable_timing=True) if timing else _new_event()
        ev.record(ld.h2d_stream)
        if timing:
            ld.copy_timing.append((t0, ev, (b - a) * 2))
        if j == len(self.pieces) - 1:
            ld._copies.append(ev)
            if len(ld._copies) > 64:
                _backlog(ld._copies)
            self.done = ev
        self.pushed += 1

    def close(self, cast_later: bool = False) -> torch.cuda.Event:
        """The last piece's copy event (there is no cast to leave for later)."""
        if self.pushed != len(self.pieces) or self.done is None:
            raise RuntimeError(f"BF16Loader pieces: {self.pushed} of {len(self.pieces)} pieces pushed")
        return self.done

    def abort(self) -> None:
        """Nothing to give back: the unit is loaded whole later."""


class GradStagingRing:
    """``depth`` pinned bf16 host slots of ``max_elems`` for gradient D2H.

    Replaces the single shared ``_cpu_grad_buffer`` of reference
    slide_fsdp.py:174-179; a slot is handed back by the update thread once
    LayerAdam has consumed it.
    """

    def __init__(self, depth: int, max_elems: int, dtype: torch.dtype = torch.bfloat16):
        self.slots = [pinned_empty(max_elems, dtype) for _ in range(depth)]
        self._free: "queue.Queue[int]" = queue.Queue()
        for i in range(depth):
            self._free.put(i)

    def acquire(self, timeout: Optional[float] = None, unit: Optional[int] = None) -> int:
        try:
            return self._free.get(timeout=timeout)
        except queue.Empty:
            raise TimeoutError("GradStagingRing.acquire: no slot released in time") from None

    def release(self, idx: int) -> None:
        self._free.put(idx)


class GradSlotRing:
    """Pinned gradient slots when one per unit does not fit the host's
    pinned memory.  Units more than twice the median unit's size (the output
    unit; a dense embedding) keep a slot of their own; the others share a
    ring of slots of the largest remaining unit, so a ring slot holds one
    decoder's gradients instead of the output unit's.  ``grow`` adds ring
    slots once the step's other pinned buffers exist.  Ring slots have ids
    0, 1, ...; a unit's own slot has the id ``("unit", u)``."""

    def __init__(self, unit_sizes: Dict[int, int], depth: int, dtype: torch.dtype = torch.bfloat16):
        sizes = sorted(unit_sizes.values())
        median = sizes[len(sizes) // 2] if sizes else 1
        self.big = {u: n for u, n in unit_sizes.items() if n > 2 * median}
        small = [n for u, n in unit_sizes.items() if u not in self.big]
        self.slot_elems = max(1, max(small) if small else max(sizes, default=1))
        self.n_small = len(small)
        self._dtype = dtype
        self.slots: Dict[Any, torch.Tensor] = {}
        for u, n in self.big.items():
            self.slots[("unit", u)] = pinned_empty(max(1, n), dtype)
        self._free: "queue.Queue[int]" = queue.Queue()
        self.depth = 0
        for _ in range(depth):
            self._publish(pinned_empty(self.slot_elems, dtype))

    def _publish(self, t: torch.Tensor) -> None:
        i = self.depth
        self.slots[i] = t
        self.depth += 1
        self._free.put(i)

    def grow(self, max_depth: int, headroom_bytes: int) -> int:
        """Pin more ring slots, up to ``max_depth``, until the host refuses;
        then give back enough of the new ones to leave ``headroom_bytes``
        pinnable for buffers allocated later.  Returns the slots added."""
        new: List[torch.Tensor] = []
        refused = False
        while self.depth + len(new) < max_depth:
            try:
                new.append(pinned_empty(self.slot_elems, self._dtype))
            except _native.NativeError as e:
                if e.status != _native.HIP_ERROR_OUT_OF_MEMORY:
                    raise
                refused = True
                break
        if refused:
            per = self.slot_elems * torch.empty((), dtype=self._dtype).element_size()
            for _ in range(min(len(new), -(-headroom_bytes // per))):
                new.pop()
        for t in new:
            self._publish(t)
        return len(new)

    def acquire(self, timeout: Optional[float] = None, unit: Optional[int] = None):
        """A ring slot (blocking), or with ``unit`` a big unit's own slot."""
        if unit is not None and unit in self.big:
            return ("unit", unit)
        try:
            return self._free.get(timeout=timeout)
        except queue.Empty:
            raise TimeoutError("GradSlotRing.acquire: no slot released in time") from None

    def own_slot(self, unit: int):
        """The unit's own slot id, or None for a unit that uses the ring."""
        return ("unit", unit) if unit in self.big else None

    def release(self, idx) -> None:
        if isinstance(idx, tuple):
            return None
        self._free.put(idx)


class GradSlotsPerUnit:
    """One pinned bf16 host slot per unit, sized to the unit.

    A unit has at most one gradient offload outstanding (its next backward
    follows its next forward, which waits for its update), so its slot is
    always free: gradient D2H never waits for the host optimizer, and
    updates may run in any order.  Costs 2 bytes of pinned host memory per
    parameter.
    """

    def __init__(self, unit_sizes: Dict[int, int], dtype: torch.dtype = torch.bfloat16):
        self.slots = {}
        for u, n in unit_sizes.items():
            self.slots[u] = pinned_empty(max(1, n), dtype)

    def acquire(self, timeout: Optional[float] = None, unit: Optional[int] = None) -> int:
        if unit not in self.slots:
            raise KeyError(f"GradSlotsPerUnit: no slot for unit {unit}")
        return unit

    def release(self, idx: int) -> None:
        return None


class PriorityUpdateExecutor:
    """One worker thread that runs queued host updates lowest priority value
    first, among those whose input is ready.

    The reference runs updates first-in first-out, i.e. in backward order
    (slide_fsdp.py:163), so the units the next forward needs first are
    updated last.  Taking the ready unit the next forward needs soonest lets
    the next forward start while later units are still being updated.  Each
    unit's update is independent of the others' within a step, so the order
    does not change any result.

    A task may carry a ``ready`` object with ``query()`` and ``synchronize()``
    (a device event marking the end of its input's production).  Inputs
    complete in submission order (one stream or engine queue), so when no
    queued task is ready the worker waits for the oldest one, never for a
    later one.

    ``gate`` (optional) is called by the worker before each pick, outside the
    lock, and may block until a resource is free (a host gradient slot); its
    result is passed to the picked task as its first argument.  The choice is
    made once the resource is there, so it goes to the most urgent task.
    """

    def __init__(self, name: str, gate: Optional[Callable[[], Any]] = None):
        self._tasks: list = []   # [priority, seq, future, fn, args, ready]
        self._cv = threading.Condition()
        self._seq = 0
        self._stop = False
        self._gate = gate
        self._thread = threading.Thread(target=self._run, name=name, daemon=True)
        self._thread.start()

    def submit(self, priority: int, fn: Callable, *args, ready=None) -> Future:
        f: Future = Future()
        with self._cv:
            if self._stop:
                raise RuntimeError("PriorityUpdateExecutor: shut down")
            self._tasks.append((priority, self._seq, f, fn, args, ready))
            self._seq += 1
            self._cv.notify()
        return f

    @staticmethod
    def _ready(t) -> bool:
        if t[5] is None:
            return True
        try:
            return bool(t[5].query())
        except BaseException:
            return True   # a failed input: the task runs and reports it

    def _pick(self):
        """Under the lock: (task, must_wait).  The lowest-priority ready task,
        else the oldest task, to be waited for outside the lock."""
        for t in sorted(self._tasks, key=lambda t: (t[0], t[1])):
            if self._ready(t):
                return t, False
        return min(self._tasks, key=lambda t: t[1]), True

    def _run(self) -> None:
        while True:
            with self._cv:
                self._cv.wait_for(lambda: self._tasks or self._stop)
                if not self._tasks:
                    return
            token, gate_error = None, None
            if self._gate is not None:
                try:
                    token = self._gate()
                except BaseException as e:  # e.g. no slot freed in time: fail the oldest task
                    gate_error = e
            with self._cv:
                if gate_error is not None:
                    task = min(self._tasks, key=lambda t: t[1])
                    self._tasks.remove(task)
                    if task[2].set_running_or_notify_cancel():
                        task[2].set_exception(gate_error)
                    continue
                task, must_wait = self._pick()
                if not must_wait:
                    self._tasks.remove(task)
            if must_wait and getattr(task[5], "poll_interval", None):
                # Readiness that other queued tasks' progress can bring about
                # (moments read back into buffers they free): pick again until
                # some task is ready instead of committing to the oldest.  If
                # none is for poll_fallback_s, run the oldest anyway (it then
                # waits for its own inputs), so progress never depends on the
                # readiness reports alone.
                deadline = time.monotonic() + task[5].poll_fallback_s
                while must_wait and time.monotonic() < deadline:
                    time.sleep(task[5].poll_interval)
                    with self._cv:
                        task, must_wait = self._pick()
                        if not must_wait:
                            self._tasks.remove(task)
                if must_wait:
                    with self._cv:
                        task = min(self._tasks, key=lambda t: t[1])
                        self._tasks.remove(task)
                    try:
                        task[5].synchronize()
                    except BaseException:
                        pass
            elif must_wait:
                try:
                    task[5].synchronize()
                except BaseException:
                    pass  # the task itself reports the failure when it runs
                with self._cv:
                    task, _ = self._pick()
                    self._tasks.remove(task)
            _, _, f, fn, args, _ = task
            if self._gate is not None:
                args = (token,) + tuple(args)
            if not f.set_running_or_notify_cancel():
                continue
            try:
                f.set_result(fn(*args))
            except BaseException as e:  # delivered to whoever waits on f
                f.set_exception(e)

    def shutdown(self, wait: bool = True) -> None:
        with self._cv:
            self._stop = True
            self._cv.notify_all()
        if wait and self._thread is not threading.current_thread():
            self._thread.join()


class _UpdateReady:
    """``query`` is true once the gradients have landed and the moments are
    in memory.  A unit's moments may wait for a buffer that another queued
    unit's update frees, so the executor must not commit to one waiting
    task: ``poll_interval`` makes it pick again until some task is ready.
    ``synchronize`` waits for the gradients only (the update reads moments
    that are still on storage itself)."""

    poll_interval = 200e-6
    poll_fallback_s = 10.0

    def __init__(self, grads_ready, optimizer, unit: int):
        self.grads_ready, self.optimizer, self.unit = grads_ready, optimizer, unit

    def query(self) -> bool:
        try:
            return ((self.grads_ready is None or self.grads_ready.query())
                    and self.optimizer.states_ready(self.unit))
        except BaseException:
            return True  # a failed copy or read: the update runs and reports it

    def synchronize(self) -> None:
        if self.grads_ready is not None:
            self.grads_ready.synchronize()


class _LinkQuiet:
    """Ready once ``first`` has completed and no host-to-device copy of a
    unit is queued.  For update work that may wait (the embedding's
    gradient-free rows): its host-memory traffic would slow the copies the
    forward is waiting for, so it runs once they have landed.  Polled by the
    executor like ``_UpdateReady``; after ``poll_fallback_s`` it runs anyway."""

    poll_interval = 200e-6
    poll_fallback_s = 10.0

    def __init__(self, first, stager):
        self.first, self.stager = first, stager

    def query(self) -> bool:
        return self.first.query() and self.stager.backlog() == 0

    def synchronize(self) -> None:
        self.first.synchronize()


def _no_slot() -> None:
    """Offload gate with one slot per unit: nothing to wait for."""
    return None


class StreamingRuntime:
    """Objects shared by all units of one model: streams, pool, stager, grad
    ring, worker threads and the optional event trace."""

    def __init__(self, device: torch.device, dtype: torch.dtype, max_param_size: int, pool_size: int,
                 stage_chunk_elems: int, stage_depth: int, grad_ring_depth: int, wait_timeout: Optional[float],
                 d2h_workgroups: int = 8, d2h_engine: str = "sdma", h2d_format: str = "fp32"):
        if d2h_engine not in ("sdma", "kernel", "copy"):
            raise ValueError("d2h_engine must be 'kernel', 'copy' or 'sdma'")
        if h2d_format not in ("fp32", "bf16"):
            raise ValueError("h2d_format must be 'fp32' or 'bf16'")
        if h2d_format == "bf16" and dtype != torch.bfloat16:
            raise ValueError("h2d_format='bf16' needs bf16 units")
        self.device = device
        # Parameter H2D: "fp32" (default) copies the fp32 masters and casts
        # them on the GPU; "bf16" copies a bf16 host copy that the optimizer
        # keeps current, half the bytes on the host link.
        self.h2d_format = h2d_format
        # Gradient D2H: "sdma" (default) hands them to SDMA engines of their
        # own through ROCr, ~50 GB/s with no shader traffic, so the backward
        # kernels beside it run at full speed; "kernel" packs them with a
        # capped-grid kernel writing into host memory (~49 GB/s, but every
        # kernel running beside a PCIe-writing kernel slows down, the GEMMs
        # ~2-4x); "copy" issues one hipMemcpyAsync per parameter, which the
        # runtime performs with a blit kernel (~18 GB/s).
        self.d2h_engine = d2h_engine
        if d2h_engine == "sdma":
            kernels.dma_init(device)
        # Host AdamW team size (0: leave the library's setting alone); see
        # set_adam_threads.
        self.adam_threads = 0
        self._adam_threads_set = 0
        # Workgroups of the kernels that write into pinned host memory (grad
        # and checkpoint offload): 8 move ~49 GB/s while the link is busy the
        # other way; more do not move more, and slow HBM-bound kernels beside
        # them (the staging cast: 1.75x with 8, 10x with 64).
        self.d2h_workgroups = d2h_workgroups
        self.h2d_stream = torch.cuda.Stream(device=device)
        self.cast_stream = torch.cuda.Stream(device=device)
        self.d2h_stream = torch.cuda.Stream(device=device)
        self.pool = LayerBufferPool(max_param_size, dtype, device, pool_size)
        if h2d_format == "bf16":
            self.stager = BF16Loader(self.h2d_stream)
        else:
            # whole-unit slots of units staged after their update: at most a
            # quarter of the device memory
            cap = torch.cuda.get_device_properties(device).total_memory // 4
            self.stager = H2DStager(device, stage_chunk_elems, stage_depth, self.h2d_stream, self.cast_stream,
                                    slot_cap_bytes=cap)
        # Gradient host slots: a ring of ``grad_ring_depth`` max-size slots,
        # or (None) one slot per unit, set up by ``init_grad_slots``.
        self.grad_ring = None if grad_ring_depth is None else GradStagingRing(grad_ring_depth, max_param_size, dtype)
        self._dtype = dtype
        # One thread issues gradient offloads (it may wait for a free host
        # slot); one thread runs the host optimizer, as the reference's
        # update executor (slide_fsdp.py:163).
        # Gradient offloads: issued by one thread, the most urgent ready unit
        # first (``init_grad_slots`` sets it up once the slots exist).
        self.offload_executor: Optional[PriorityUpdateExecutor] = None
        self.update_executor = PriorityUpdateExecutor("sf-update")
        # Units with their own device buffer are staged for the next forward
        # by the update thread, right after their update.
        self.stage_after_update = False
        # Queue priority of a unit's update (lower runs first); the model sets
        # it to the unit's position in the next forward.
        self.update_priority: Callable[[int], int] = lambda unit: unit
        # Elements per piece of a unit's update (0: whole units).  Gradients
        # come back in pieces, the host AdamW starts on the first piece that
        # has landed, and each updated piece is copied to the device while
        # the next one is being updated.
        self.piece_elems = 0
        # Units staged after their update (fp32 H2D) are cast where they are
        # next used, on that stream between its kernels, instead of on the
        # cast stream as soon as their copy lands.
        self.cast_at_use = False
        self.wait_timeout = wait_timeout
        self.trace: Optional[List[Tuple]] = None
        self._trace_lock = threading.Lock()
        # Optional host timeline: (perf_counter, thread name, event, unit).
        self.timeline: Optional[list] = None
        self.d2h_timing: Optional[list] = None
        # Test hook: when a dict, each update stores {unit: (host grads, fp32
        # master before the update)} and each gradient offload stores
        # {("device_grads", unit): [param.grad clones]}, for checking the
        # pack and the update against the oracle.
        self.capture: Optional[dict] = None

    def set_adam_threads(self) -> None:
        """Team size of the next host update (update thread).  With two or
        more units' copies still queued for the host-to-device link, the
        AdamW is ahead of the link, the step's bottleneck: it then runs on
        half of its threads, which leaves host memory bandwidth and cores to
        the copies and to the threads that feed the GPU.  Measured, Llama-3-8B
        step, same box: 745-750 ms against 797-801 ms with every update on
        all threads; a threshold of one queued unit 756-760 ms, of three
        816 ms; 6 threads 764-768 ms, 10 threads 783 ms.  With bf16 H2D (half
        the link bytes) the AdamW is the bottleneck and keeps all its threads
        (yielding there measured 1.5 % slower)."""
        if not self.adam_threads or self.h2d_format != "fp32":
            return
        few = self.stager.backlog() >= 2
        n = max(1, (self.adam_threads + 1) // 2) if few else self.adam_threads
        if n != self._adam_threads_set:
            _cpu_adam.set_num_threads(n)
            self._adam_threads_set = n

    def init_grad_slots(self, unit_sizes: Dict[int, int], fallback_depth: int = 3) -> None:
        """One pinned slot per unit; if the host cannot pin that much (the
        driver caps pinned memory well below the host's RAM on some
        machines), a ring of ``fallback_depth`` slots of the largest unit.
        Then the offload thread: with a ring it takes a free slot first and
        then the most urgent unit whose gradients are complete (the others
        wait in HBM); with per-unit slots it never waits for a slot."""
        if self.grad_ring is None:
            self._alloc_grad_slots(unit_sizes, fallback_depth)
        if self.offload_executor is None:
            ring = self.grad_ring
            if isinstance(ring, GradSlotsPerUnit):
                gate = _no_slot       # the task takes its unit's own slot
            else:
                gate = lambda: ring.acquire(timeout=self.wait_timeout)  # noqa: E731
            self.offload_executor = PriorityUpdateExecutor("sf-offload", gate=gate)

    def _alloc_grad_slots(self, unit_sizes: Dict[int, int], fallback_depth: int) -> None:
        try:
            self.grad_ring = GradSlotsPerUnit(unit_sizes, self._dtype)
            return
        except _native.NativeError as e:
            if e.status != _native.HIP_ERROR_OUT_OF_MEMORY:
                raise
        # Outside the handler: the traceback no longer holds the slots pinned
        # so far, so they are released before the ring is pinned.
        need = 2 * sum(unit_sizes.values())
        ring = GradSlotRing(unit_sizes, fallback_depth, self._dtype)
        print(f"SlideFSDP: {need / 1e9:.1f} GB of pinned gradient slots (one per unit) do not fit; "
              f"using {len(ring.big)} slot(s) of their own for the largest units and a ring of "
              f"{fallback_depth} slots of {2 * ring.slot_elems / 1e9:.2f} GB (grown after the first step)",
              flush=True)
        self.grad_ring = ring

    def log(self, *event) -> None:
        if self.trace is not None:
            with self._trace_lock:
                self.trace.append(tuple(event))

    def mark(self, what: str, unit: int) -> None:
        if self.timeline is not None:
            self.timeline.append((time.perf_counter(), threading.current_thread().name, what, unit))

    def shutdown(self) -> None:
        if self.offload_executor is not None:
            self.offload_executor.shutdown(wait=True)
        self.update_executor.shutdown(wait=True)

    def release_slots(self, states) -> None:
        """Give back the whole-unit slots of stagings not yet cast (their units
        are then staged from the master if used again) and free the pool's
        buffers once the copy and cast streams have drained."""
        slots = getattr(self.stager, "slots", None)
        if slots is None:
            return
        for st in states:
            with st._prefetch_lock:
                pre = st._prefetched
                if pre is not None and isinstance(pre[1], PendingCast):
                    st._prefetched = None
                else:
                    pre = None
            if pre is not None:
                self.stager.drop_pending(pre[1])
            st._drop_pending_cast()
        self.h2d_stream.synchronize()
        self.cast_stream.synchronize()
        slots.release()


class LayerRuntimeState(nn.Module):
    """Runtime of one unit: fp32 pinned master, device residency, gradient
    offload and the asynchronous host update.

    Reference layer_state.py:105-467; method names and meanings are kept:
    ``to_device_async``, ``wait_for_h2d``, ``to_offload_async``,
    ``wait_for_d2h``, ``update_params``, ``wait_for_update``.
    """

    def __init__(self, layer: nn.Module, layer_idx: int, config, runtime: StreamingRuntime,
                 layer_optimizer: Any, is_last_layer: bool = False):
        super().__init__()
        self.layer = layer
        self.layer_idx = layer_idx
        self.config = config
        self.runtime = runtime
        self.buffer_pool = runtime.pool
        self.layer_optimizer = layer_optimizer
        self.is_last_layer = is_last_layer

        self.update_finished = threading.Event()
        self.update_finished.set()
        self.update_lock = threading.Lock()
        self._h2d_done: Optional[torch.cuda.Event] = None
        self._d2h_future: Optional[Future] = None
        self._update_future: Optional[Future] = None
        self._current_gpu_cache: Optional[Dict[str, Any]] = None
        # A unit of its own (``make_resident``): loaded in the forward and
        # kept on the device through the backward, never taken from the pool.
        self._own_unit: Optional[Dict[str, Any]] = None
        # Row-sparse embedding (``enable_row_sparse``): only the batch's rows
        # cross the host link, in both directions.
        self.row_sparse = False
        # Own unit already staged with the next step's weights by the update
        # thread (``stage_for_next_forward``): (unit, copy-and-cast event).
        self._prefetched: Optional[Tuple[Dict[str, Any], torch.cuda.Event]] = None
        self._prefetch_lock = threading.Lock()
        self._plan_key: Optional[int] = None
        self._plan = None
        # Own unit bound with its weights copied but not cast yet: cast by
        # ``wait_for_h2d`` on the stream about to use the unit.
        self._pending_cast: Optional[PendingCast] = None
        self._post_called = False
        self._bwd_armed = False
        self._bwd_compute_done = False
        self._grads_offloaded = False

        params = list(self.layer.parameters())
        self.total_size = sum(p.numel() for p in params)
        # Units whose backward does not read their parameters skip the reload
        # before their backward (the reference reloads every unit,
        # slide_fsdp.py:443-444).
        self.backward_reads_params = not isinstance(self.layer, nn.Embedding)
        # The fp32 master is the H2D source with fp32 H2D and must be pinned;
        # with bf16 H2D only the host optimizer touches it, so it stays in
        # pageable memory and the pinned budget (which the driver caps well
        # below the host's RAM on some machines) goes to the bf16 copy.
        if runtime.h2d_format == "bf16":
            self._cpu_params_flat = torch.empty(self.total_size, dtype=torch.float32)
        else:
            self._cpu_params_flat = pinned_empty(self.total_size, torch.float32)
        self._param_maps: "OrderedDict[str, Tuple[int, torch.Size, int]]" = OrderedDict()
        self._param_views: "OrderedDict[str, torch.Tensor]" = OrderedDict()
        self._params: List[nn.Parameter] = []
        self._init_param_views()
        # bf16 H2D: a pinned bf16 copy of the master, rewritten by every update.
        self._cpu_params_bf16: Optional[torch.Tensor] = None
        if runtime.h2d_format == "bf16":
            try:
                self._cpu_params_bf16 = pinned_empty(self.total_size, torch.bfloat16)
            except _native.NativeError as e:
                if e.status != _native.HIP_ERROR_OUT_OF_MEMORY:
                    raise
                raise RuntimeError(
                    "h2d_format='bf16' keeps a pinned bf16 copy of every master (2 bytes per parameter) "
                    "and this host cannot pin that much"
                ) from e
            self.refresh_host_copy()
        self._grad_params = [p for p in self._params if p.requires_grad]
        self._grads_seen = 0
        self._grad_lock = threading.Lock()
        if self.layer_optimizer is not None:
            self.layer_optimizer.add_layer_params(layer_idx, self._params)

    # ------------------------------------------------------------------
    def _init_param_views(self) -> None:
        """Flatten in ``named_parameters()`` order into the pinned fp32 master and
        point every ``param.data`` at its view (reference layer_state.py:240-264)."""
        with torch.no_grad():
            offset = 0
            for name, param in self.layer.named_parameters():
                size = param.numel()
                self._param_maps[name] = (offset, param.shape, size)
                view = self._cpu_params_flat[offset:offset + size].view(param.shape)
                view.copy_(param.data)
                self._param_views[name] = view
                param.data = view
                param.grad = None
                self._params.append(param)
                offset += size

    def _named(self):
        return zip(self._param_maps.items(), self._params)

    def refresh_host_copy(self) -> None:
        """Recompute the bf16 host copy from the fp32 master (bf16 H2D only)
        and drop a staging made for the next forward.  Updates keep both
        current; call this after writing the master directly."""
        with self._prefetch_lock:
            old, self._prefetched = self._prefetched, None
        if old is not None and isinstance(old[1], PendingCast):
            self.runtime.stager.drop_pending(old[1])
        if self._cpu_params_bf16 is not None and self.total_size:
            _cpu_adam.cast_f32_bf16(self._cpu_params_flat, self._cpu_params_bf16)

    def stage_for_next_forward(self) -> None:
        """Stage the freshly updated master into this unit's own device buffer
        (update thread, right after the update).  The copy starts during the
        backward, when the host-to-device direction of the link is otherwise
        idle, instead of in the next forward; the cast waits for the buffer's
        last reader (the unit's backward).  Same bits as staging in the
        forward: the master does not change before the next update."""
        unit = self._own_unit
        if unit is None or self._current_gpu_cache is not None or self.row_sparse:
            return
        stager = self.runtime.stager
        done = None
        if self._cpu_params_bf16 is not None:
            done = stager.load(self._cpu_params_bf16, unit["param"], unit["ready"])
        elif self.runtime.cast_at_use:
            done = stager.copy_for_later(self._cpu_params_flat, unit["ready"])
        if done is None:
            done = stager.finish(stager.begin(self._cpu_params_flat), unit["param"], unit["ready"])
        self._set_prefetched(unit, done)
        self.runtime.mark("staged_after_update", self.layer_idx)

    def _set_prefetched(self, unit: Dict[str, Any], done) -> None:
        """Record the staging of the own unit for the next forward: its cast's
        completion event, or a ``PendingCast``."""
        with self._prefetch_lock:
            old, self._prefetched = self._prefetched, (unit, done)
        if old is not None and isinstance(old[1], PendingCast):
            self.runtime.stager.drop_pending(old[1])

    def _drop_pending_cast(self) -> None:
        pc, self._pending_cast = self._pending_cast, None
        if pc is not None:
            self.runtime.stager.drop_pending(pc)

    def _bind_device_views(self, unit: Dict[str, Any]) -> None:
        buf = unit["param"]
        for (name, (off, shape, size)), p in self._named():
            p.data = buf[off:off + size].view(shape)
            p.grad = None

    def _bind_host_views(self) -> None:
        for (name, _), p in self._named():
            p.data = self._param_views[name]
            p.grad = None

    # ------------------------------------------------------------------
    def to_device_async(self, is_backward: bool = False) -> None:
        """Start loading this unit; returns once the work is enqueued.

        Waits on the host only for this unit's previous update (so the master
        is current) and then for a free pool unit; the fp32 copies into the
        staging ring are issued before the pool wait, so the host link keeps
        streaming while an earlier unit is still busy.
        """
        if self.row_sparse:
            # rows are gathered by the lookup itself (gather_rows); the
            # backward of a lookup reads no weights
            self.runtime.log("h2d", self.layer_idx, is_backward)
            return
        if self._current_gpu_cache is not None:
            return  # already resident (last decoder / output / own unit)
        self.wait_for_update()
        # Checked after the update: the update thread stages an own unit for
        # the next forward as the last part of the update task.
        with self._prefetch_lock:
            pre, self._prefetched = self._prefetched, None
        if pre is not None:
            unit, done = pre
            self._drop_pending_cast()
            if isinstance(done, PendingCast):
                self._pending_cast, self._h2d_done = done, None
            else:
                self._h2d_done = done
            self._bind_unit(unit, is_backward)
            return
        stager = self.runtime.stager
        # The backward of an embedding never reads its weights (its gradient
        # depends only on the indices), so no copy or cast is needed then.
        skip = is_backward and not self.backward_reads_params
        if self._cpu_params_bf16 is not None:
            unit = self._acquire_unit()
            self._h2d_done = unit["ready"] if skip else stager.load(self._cpu_params_bf16, unit["param"], unit["ready"])
            self._bind_unit(unit, is_backward)
            return
        ticket = None if skip else stager.begin(self._cpu_params_flat)
        try:
            unit = self._acquire_unit()
        except BaseException:
            if ticket is not None:
                stager.finish(ticket, self._dummy_dst(), None)
            raise
        if ticket is None:
            self._h2d_done = unit["ready"]   # keep the release fence of the unit
        else:
            self._h2d_done = stager.finish(ticket, unit["param"], unit["ready"])
        self._bind_unit(unit, is_backward)

    def make_resident(self, buffer: torch.Tensor) -> None:
        """Give this unit a device buffer of its own (at least ``total_size``
        elements of the pool dtype).  Its weights are then loaded once per
        step, in the forward, and stay on the device until its backward has
        finished: the backward reload of the reference (slide_fsdp.py:443-444)
        is skipped.  The staged bits are the same either way, since the master
        only changes in the update that follows the backward."""
        if buffer.numel() < self.total_size or buffer.dtype != self.buffer_pool.dtype:
            raise ValueError("make_resident: buffer too small or of the wrong dtype")
        if self._current_gpu_cache is not None:
            raise RuntimeError("make_resident: unit is loaded")
        self._own_unit = {"param": buffer, "grad": None, "ready": None}

    @property
    def resident_across_steps(self) -> bool:
        return self._own_unit is not None

    def _acquire_unit(self) -> Dict[str, Any]:
        if self._own_unit is not None:
            return self._own_unit
        return self.buffer_pool.acquire(timeout=self.runtime.wait_timeout)

    def _release_unit(self, unit: Dict[str, Any]) -> None:
        if unit is not self._own_unit:
            self.buffer_pool.release(unit)

    def _bind_unit(self, unit: Dict[str, Any], is_backward: bool) -> None:
        unit["ready"] = None
        self._bind_device_views(unit)
        self._current_gpu_cache = unit
        self._bwd_compute_done = False
        self._grads_offloaded = False
        self.runtime.log("h2d", self.layer_idx, is_backward)
        self.runtime.mark("h2d_issued", self.layer_idx)

    def _dummy_dst(self) -> torch.Tensor:
        # Only used to drain a staging ticket after a failed acquire: casts
        # into a scratch buffer so the ring's slot events stay consistent.
        return torch.empty(self.total_size, dtype=torch.bfloat16, device=self.runtime.device)

    def wait_for_h2d(self, timeout: Optional[float] = None) -> None:
        """Make the current stream wait for this unit's load (no host block).
        A unit whose weights were copied but not cast is cast here, on the
        current stream, after its copy."""
        pc = self._pending_cast
        if pc is not None:
            unit = self._current_gpu_cache
            if unit is None:
                raise RuntimeError(f"unit {self.layer_idx}: a pending cast without a bound unit")
            self._pending_cast = None
            self._h2d_done = self.runtime.stager.cast_pending(pc, unit["param"], torch.cuda.current_stream())
        if self._h2d_done is not None:
            torch.cuda.current_stream().wait_event(self._h2d_done)

    def is_resident(self) -> bool:
        return self._current_gpu_cache is not None

    # ------------------------------------------------------------------
    def to_offload_async(self, is_backward: bool = False, prev_update=None) -> None:
        """Release this unit after its forward (``is_backward=False``) or offload
        its gradients after its backward (``is_backward=True``).

        Forward: the unit becomes reusable once the current stream has passed
        this point.  Backward: the gradients are handed to the offload thread,
        which packs them with one kernel straight into a pinned host slot on
        ``d2h_stream``, and the update is queued behind it.  The pool unit is
        released separately, by ``mark_backward_compute_done`` and this call
        together (whichever comes last), because the unit's weights may still
        be read by backward kernels enqueued after its last gradient.
        ``prev_update`` is accepted for signature compatibility; the grad ring
        makes it unnecessary.
        """
        unit = self._current_gpu_cache
        if unit is None:
            return
        cur = torch.cuda.current_stream()
        if not is_backward:
            if unit is self._own_unit:
                return  # stays loaded for the backward
            ev = _new_event()
            ev.record(cur)
            unit["ready"] = ev
            self._bind_host_views()
            self._current_gpu_cache = None
            self.buffer_pool.release(unit)
            return

        grads, missing = [], []
        for (name, (off, shape, size)), p in self._named():
            g = p.grad
            if g is None:
                missing.append((off, size))
                continue
            if g.dtype != unit["param"].dtype or g.device != unit["param"].device:
                raise RuntimeError(f"unit {self.layer_idx}: grad of {name} is {g.dtype} on {g.device}, "
                                   f"expected {unit['param'].dtype} on {unit['param'].device}")
            grads.append((g.detach().contiguous().reshape(-1), off))
        if self.runtime.capture is not None:
            self.runtime.capture[("device_grads", self.layer_idx)] = [
                None if p.grad is None else p.grad.detach().clone() for p in self._params]
        grad_ready = _new_event()
        grad_ready.record(cur)
        # The cast issued last before these gradients existed (the next unit's
        # load); the pack is ordered behind it, not behind later ones.
        cast_fence = self.runtime.stager.last_cast_done
        for p in self._params:
            p.grad = None
        self.update_finished.clear()
        self.runtime.log("d2h", self.layer_idx)
        self.runtime.mark("post_backward", self.layer_idx)
        rt = self.runtime
        self._d2h_future = rt.offload_executor.submit(rt.update_priority(self.layer_idx), self._d2h_task,
                                                      grads, missing, grad_ready, cast_fence, ready=grad_ready)
        self._grads_offloaded = True
        self._maybe_release_after_backward()

    def mark_backward_compute_done(self) -> None:
        """Every backward kernel that reads this unit's weights has been
        enqueued on the current stream (called when the gradient has flowed
        past the unit's first operation)."""
        if self._current_gpu_cache is None:
            return
        self._bwd_compute_done = True
        self._maybe_release_after_backward()

    def _maybe_release_after_backward(self) -> None:
        unit = self._current_gpu_cache
        if unit is None or not (self._bwd_compute_done and self._grads_offloaded):
            return
        ev = _new_event()
        ev.record(torch.cuda.current_stream())
        unit["ready"] = ev
        self._bind_host_views()
        self._current_gpu_cache = None
        self._release_unit(unit)

    def _piece_plan(self):
        """``(bounds, param_ranges)``: the flat ``[a, b)`` pieces this unit's
        update runs in and, per piece, its ``(param, lo, hi)`` ranges; None
        when the unit is one piece."""
        pe = int(self.runtime.piece_elems or 0)
        if self._plan_key != pe:
            named = list(self._named())
            spans = [(off, size) for (_, (off, _, size)), _ in named]
            plan = None
            if pe > 0 and all(off == sum(sz for _, sz in spans[:i]) for i, (off, _) in enumerate(spans)):
                bounds = split_into_pieces([sz for _, sz in spans], pe)
                if len(bounds) > 1:
                    params = [p for _, p in named]
                    plan = (bounds, [[(params[i], lo, hi) for i, lo, hi in overlap_ranges(spans, a, b)]
                                     for a, b in bounds])
            self._plan_key, self._plan = pe, plan
        return self._plan

    def _open_staging_pieces(self, bounds):
        """``(unit, piece stream)`` to stage the unit's own buffer piece by
        piece during its update, or None where ``stage_for_next_forward``
        would not stage it."""
        unit = self._own_unit
        if unit is None or self._current_gpu_cache is not None or self.row_sparse:
            return None
        stager = self.runtime.stager
        host = self._cpu_params_bf16 if self._cpu_params_bf16 is not None else self._cpu_params_flat
        stream = stager.open_pieces(host, unit["param"], unit["ready"], bounds)
        return None if stream is None else (unit, stream)

    def _d2h_task(self, slot, grads, missing, grad_ready, cast_fence) -> None:
        """Offload thread: copy this unit's gradients into a host slot, then
        queue the update.  ``slot`` is the ring slot the thread's gate took,
        or None with one slot per unit (the unit's own is taken here)."""
        rt = self.runtime
        if slot is None:
            slot = rt.grad_ring.acquire(timeout=rt.wait_timeout, unit=self.layer_idx)
        else:
            own = getattr(rt.grad_ring, "own_slot", None)
            if own is not None and own(self.layer_idx) is not None:
                # a unit with a slot of its own hands the ring slot back
                rt.grad_ring.release(slot)
                slot = own(self.layer_idx)
        rt.mark("d2h_task", self.layer_idx)
        rt.mark("slot", self.layer_idx)
        try:
            host = rt.grad_ring.slots[slot]
            pairs = [(g, host[off:off + g.numel()]) for g, off in grads]
            if rt.d2h_engine == "sdma":
                # The gradients must be complete before an SDMA engine reads
                # them (the copy is not stream-ordered): wait here, on this
                # worker thread, then hand the copy to the engine.
                grad_ready.synchronize()
                rt.mark("grad_ready", self.layer_idx)
                plan = self._piece_plan()
                if plan is None:
                    handles = [kernels.dma_copy_d2h(pairs)]
                else:
                    # one copy per piece, in update order: the update starts
                    # once the first has landed
                    spans = [(off, g.numel()) for g, off in grads]
                    handles = []
                    for a, b in plan[0]:
                        sub = [(grads[i][0][lo:hi], host[grads[i][1] + lo:grads[i][1] + hi])
                               for i, lo, hi in overlap_ranges(spans, a, b)]
                        handles.append(kernels.dma_copy_d2h(sub) if sub else None)
                rt.mark("dma_issued", self.layer_idx)
                done = None
                dma_ready = [None if h is None else kernels.DmaReady(h) for h in handles]
                handle = handles
            else:
                rt.d2h_stream.wait_event(grad_ready)
                if cast_fence is not None:
                    rt.d2h_stream.wait_event(cast_fence)
                timing = rt.d2h_timing is not None
                if timing:
                    t0 = torch.cuda.Event(enable_timing=True)
                    t0.record(rt.d2h_stream)
                if rt.d2h_engine == "copy":
                    # stream-ordered DMA copies, one per parameter
                    for g, h in pairs:
                        kernels.memcpy_async(h, g, rt.d2h_stream)
                else:
                    kernels.copy_segs_b16(pairs, rt.d2h_stream, max_workgroups=rt.d2h_workgroups)
                for g, _ in grads:
                    g.record_stream(rt.d2h_stream)
                done = torch.cuda.Event(enable_timing=True) if timing else _new_event()
                done.record(rt.d2h_stream)
                if timing:
                    rt.d2h_timing.append((t0, done, 2 * sum(g.numel() for g, _ in grads)))
                handle = None
        except BaseException:
            rt.grad_ring.release(slot)
            self.update_finished.set()
            raise
        nbytes = 2 * sum(g.numel() for g, _ in grads)
        # With SDMA the gradient tensors stay referenced until the copy is
        # waited for; the caching allocator cannot hand them out before then.
        keep = grads if handle is not None else None
        del grads, pairs
        if handle is None:
            ready = done
        else:
            ready = next((d for d in dma_ready if d is not None), None)
        self._update_future = rt.update_executor.submit(rt.update_priority(self.layer_idx), self._do_update,
                                                        slot, done, missing, None if handle is None else dma_ready,
                                                        keep, nbytes, ready=self._update_ready(ready))

    def _update_ready(self, grads_ready):
        """Readiness of this unit's update: its gradients on the host and,
        with optimizer moments on storage, the moments read back (whose read
        is queued here, in the order the gradients land)."""
        opt = self.layer_optimizer
        if opt is None or getattr(opt, "offloader", None) is None:
            return grads_ready
        opt.prefetch_states(self.layer_idx, self.runtime.update_priority(self.layer_idx))
        return _UpdateReady(grads_ready, opt, self.layer_idx)

    def wait_for_d2h(self, timeout: Optional[float] = None) -> None:
        """Wait until the gradient offload has been issued (and re-raise its
        errors).  Unlike the reference (layer_state.py:407-408), errors of
        finished tasks are not swallowed."""
        f = self._d2h_future
        if f is not None:
            f.result(timeout=timeout)

    # ------------------------------------------------------------------
    def _master_views(self) -> Dict[nn.Parameter, torch.Tensor]:
        return {p: self._param_views[name] for (name, _), p in self._named()}

    def _bf16_views(self) -> Optional[Dict[nn.Parameter, torch.Tensor]]:
        if self._cpu_params_bf16 is None:
            return None
        return self._grad_views(self._cpu_params_bf16)

    def _grad_views(self, host: torch.Tensor) -> Dict[nn.Parameter, torch.Tensor]:
        views = {}
        for (name, (off, shape, size)), p in self._named():
            views[p] = host[off:off + size].view(shape)
        return views

    # ------------------------------------------------------------------
    # Row-sparse embedding unit
    def enable_row_sparse(self) -> None:
        """Move only the rows a batch uses, for an ``nn.Embedding`` unit.

        Forward: ``gather_rows`` reads the batch's rows straight from the
        pinned host table (fp32 master, or its bf16 copy) with one kernel and
        rounds them to bf16: the lookup's output, bit for bit, without staging
        the table (reference layer_state.py:296-314 stages all of it, 2 or 4
        bytes per parameter).  Backward: ``offload_rows`` computes the dense
        table gradient on the device as the lookup's own backward does and
        sends only the batch's rows to host; the host AdamW then updates the
        whole table with zero gradient elsewhere (``sf_adam_update_rows``),
        which is the dense update's result."""
        emb = self.layer
        if not isinstance(emb, nn.Embedding) or emb.max_norm is not None or emb.scale_grad_by_freq or emb.sparse:
            raise ValueError("enable_row_sparse: a plain nn.Embedding unit is required")
        V, H = emb.weight.shape
        if H % 16 != 0 or len(self._params) != 1:
            raise ValueError("enable_row_sparse: the row length must be a multiple of 16")
        self.row_sparse = True
        self._rows_shape = (V, H)
        self._bad_ids = pinned_empty(1, torch.int32)
        self._bad_ids.zero_()
        self._rows_host: Optional[torch.Tensor] = None
        self._ids_host: Optional[torch.Tensor] = None
        # The batch's ids on the host, copied at the lookup (pinned, event),
        # for the early part of the update; the early part itself, once queued.
        self._ids_early_host: Optional[torch.Tensor] = None
        self._lookup_ids: Optional[Tuple[torch.Tensor, torch.cuda.Event]] = None
        self._early: Optional[Dict[str, Any]] = None

    def _host_table(self) -> torch.Tensor:
        V, H = self._rows_shape
        src = self._cpu_params_bf16 if self._cpu_params_bf16 is not None else self._cpu_params_flat
        return src.view(V, H)

    def gather_rows(self, ids: torch.Tensor) -> torch.Tensor:
        """Forward lookup: [*ids.shape, H] bf16 rows of the current master."""
        self.wait_for_update()
        V, H = self._rows_shape
        flat = ids.reshape(-1)
        if flat.dtype != torch.int64:
            flat = flat.long()
        if not flat.is_contiguous():
            flat = flat.contiguous()
        out = torch.empty(tuple(ids.shape) + (H,), dtype=torch.bfloat16, device=self.runtime.device)
        # The flag's previous writer (last step's lookup) finished before that
        # step's update, which wait_for_update has just waited for.
        self._bad_ids.zero_()
        kernels.gather_rows(self._host_table(), flat, out.view(-1, H), bad=self._bad_ids,
                            stream=torch.cuda.current_stream())
        self._copy_lookup_ids(flat)
        self._bwd_compute_done = False
        self._grads_offloaded = False
        self.runtime.log("h2d", self.layer_idx, False)
        self.runtime.mark("h2d_issued", self.layer_idx)
        return out

    def _copy_lookup_ids(self, flat: torch.Tensor) -> None:
        """Copy the batch's ids to pinned host memory on the D2H stream, for
        the early part of this step's update.  The buffer's previous reader
        (last step's update) finished before this lookup, which waited for
        it."""
        rt = self.runtime
        ntok = flat.numel()
        if self._ids_early_host is None or self._ids_early_host.numel() < ntok:
            self._ids_early_host = pinned_empty(max(ntok, 1), torch.int64)
        ready = _new_event()
        ready.record(torch.cuda.current_stream())
        rt.d2h_stream.wait_event(ready)
        kernels.memcpy_async(self._ids_early_host[:ntok], flat, rt.d2h_stream)
        flat.record_stream(rt.d2h_stream)
        copied = _new_event()
        copied.record(rt.d2h_stream)
        self._lookup_ids = (self._ids_early_host[:ntok], copied)

    def start_early_update(self) -> None:
        """Queue the part of this step's update that needs no gradient: the
        table rows the batch did not touch (zero gradient) get their AdamW
        update now, at the lowest priority, so the host AdamW does it while
        it would otherwise wait for the backward's first gradients; the
        batch's rows follow once their gradient has landed (``step_rows_early``
        then ``step_rows``: the bits of the whole update).  It waits for the
        host link to have no unit copy queued, so that its host-memory traffic
        does not slow the copies the forward is waiting for.  Called by the
        model right before its backward, which is then certain to reach the
        lookup (not in the reference, whose update of the whole table waits
        for the gradient)."""
        rt = self.runtime
        opt = self.layer_optimizer
        lookup, self._lookup_ids = self._lookup_ids, None
        if (not self.row_sparse or lookup is None or opt is None or not getattr(opt, "reference_order", False)
                or not self.layer.weight.requires_grad):
            return
        if getattr(opt, "offloader", None) is not None:
            # moments on storage: the two parts would read the table's moments
            # back twice, and that step is bound by storage, not by this wait
            return
        ids, copied = lookup
        early = {"ids": ids, "ready": copied, "state": "queued"}
        self._early = early
        early["future"] = rt.update_executor.submit(EARLY_UPDATE_PRIORITY, self._do_update_rows_early, early,
                                                    ready=_LinkQuiet(copied, rt.stager))

    def _do_update_rows_early(self, early: Dict[str, Any]) -> bool:
        """Update thread: the early part queued by ``start_early_update``
        (nothing if the late part has already run it)."""
        if early["state"] != "queued":
            return False
        rt = self.runtime
        V, H = self._rows_shape
        early["ready"].synchronize()
        ids = early["ids"]
        if ids.numel() and (int(ids.min()) < 0 or int(ids.max()) >= V):
            early["state"] = "skipped"   # the late part raises for these ids
            return False
        rt.mark("early_update_start", self.layer_idx)
        slot = torch.full((V,), _native.SF_ROW_ZERO, dtype=torch.int64)
        slot[ids] = _native.SF_ROW_SKIP
        if rt.capture is not None:
            early["master_before"] = self._cpu_params_flat.clone()
        rt.set_adam_threads()
        with self.update_lock:
            early["state"] = "failed"
            self.layer_optimizer.step_rows_early(self.layer_idx, slot, param_view=self._cpu_params_flat.view(V, H),
                                                 bf16_view=None if self._cpu_params_bf16 is None
                                                 else self._cpu_params_bf16.view(V, H))
            early["state"] = "applied"
        rt.mark("early_update_done", self.layer_idx)
        return True

    def offload_rows(self, grad_out: torch.Tensor, ids: torch.Tensor) -> None:
        """Backward of the lookup: dense table gradient on the device (as the
        lookup's backward computes it), its batch rows to pinned host slots,
        then the update is queued."""
        rt = self.runtime
        V, H = self._rows_shape
        flat = ids.reshape(-1)
        ntok = flat.numel()
        pad = self.layer.padding_idx if self.layer.padding_idx is not None else -1
        # ids outside the table were flagged by the lookup (the update raises
        # for them); clamped here so that the dense backward never indexes
        # outside the table.  Valid ids are unchanged.
        dense = torch.ops.aten.embedding_dense_backward(grad_out.reshape(ntok, H), flat.clamp(0, V - 1), V, pad,
                                                        False)
        if rt.capture is not None:
            rt.capture[("device_grads", self.layer_idx)] = [dense.detach().clone().view(V, H)]
        if self._rows_host is None or self._rows_host.shape[0] < ntok:
            self._rows_host = pinned_empty((ntok, H), torch.bfloat16)
            self._ids_host = pinned_empty(ntok, torch.int64)
        grad_ready = _new_event()
        grad_ready.record(torch.cuda.current_stream())
        with self._grad_lock:
            self._post_called = True
            self._bwd_armed = False
        self.update_finished.clear()
        rt.log("d2h", self.layer_idx)
        rt.mark("post_backward", self.layer_idx)
        rt.d2h_stream.wait_event(grad_ready)
        kernels.gather_rows(dense, flat, self._rows_host[:ntok], stream=rt.d2h_stream,
                            max_workgroups=rt.d2h_workgroups)
        kernels.memcpy_async(self._ids_host[:ntok], flat, rt.d2h_stream)
        dense.record_stream(rt.d2h_stream)
        flat.record_stream(rt.d2h_stream)
        done = _new_event()
        done.record(rt.d2h_stream)
        self._grads_offloaded = True
        self._bwd_compute_done = True
        self._update_future = rt.update_executor.submit(rt.update_priority(self.layer_idx), self._do_update_rows,
                                                        done, ntok, ready=self._update_ready(done))

    def _do_update_rows(self, d2h_done: torch.cuda.Event, ntok: int) -> bool:
        rt = self.runtime
        V, H = self._rows_shape
        try:
            rt.mark("update_start", self.layer_idx)
            d2h_done.synchronize()
            if int(self._bad_ids[0]) != 0:
                raise ValueError(f"embedding unit {self.layer_idx}: input ids outside [0, {V})")
            ids = self._ids_host[:ntok]
            rows = self._rows_host[:ntok]
            early, self._early = self._early, None
            if early is not None and early["state"] == "queued":
                self._do_update_rows_early(early)   # not run yet: now, on this thread
            applied = early is not None and early["state"] == "applied"
            if early is not None and early["state"] == "failed":
                raise RuntimeError(f"embedding unit {self.layer_idx}: the early part of the update failed")
            row_slot = torch.full((V,), _native.SF_ROW_SKIP if applied else _native.SF_ROW_ZERO, dtype=torch.int64)
            row_slot[ids] = torch.arange(ntok, dtype=torch.int64)
            if rt.capture is not None:
                dense = torch.zeros(V, H, dtype=rows.dtype)
                dense[ids] = rows
                before = early["master_before"] if applied else self._cpu_params_flat.clone()
                rt.capture[self.layer_idx] = (dense.view(-1), before)
            rt.set_adam_threads()
            with self.update_lock:
                if self.layer_optimizer is not None:
                    self.layer_optimizer.step_rows(self.layer_idx, row_slot, rows,
                                                   param_view=self._cpu_params_flat.view(V, H),
                                                   bf16_view=None if self._cpu_params_bf16 is None
                                                   else self._cpu_params_bf16.view(V, H))
            rt.mark("adam_done", self.layer_idx)
        finally:
            self.update_finished.set()
        return True

    def _do_update(self, slot: int, d2h_done: Optional[torch.cuda.Event], missing: List[Tuple[int, int]],
                   dma_ready=None, keep=None, nbytes: int = 0) -> bool:
        """Update thread: the unit's AdamW from its host gradient slot, then
        (own units) its staging for the next forward.  ``dma_ready`` holds the
        SDMA copies of the gradients, one per piece of ``_piece_plan`` (or one
        for the unit); piece ``j`` is updated once copy ``j`` has landed, and
        its new weights are copied to the device while piece ``j + 1`` is
        updated (the cast follows the unit's last piece)."""
        rt = self.runtime
        chunks = list(dma_ready) if dma_ready is not None else []
        state = {"waited": 0, "t0": None, "t1": None}

        def wait_chunks(upto: int) -> None:
            while state["waited"] < len(chunks) and state["waited"] <= upto:
                ch = chunks[state["waited"]]
                state["waited"] += 1
                if ch is None:
                    continue
                t0, t1 = ch.release()
                if t1 > t0:
                    state["t0"] = t0 if state["t0"] is None else min(state["t0"], t0)
                    state["t1"] = t1 if state["t1"] is None else max(state["t1"], t1)
                if state["waited"] == 1:
                    rt.mark("dma_done", self.layer_idx)

        try:
            rt.mark("update_start", self.layer_idx)
            if d2h_done is not None:
                d2h_done.synchronize()
            plan = self._piece_plan() if self.layer_optimizer is not None else None
            if plan is None or len(chunks) not in (0, len(plan[0])):
                wait_chunks(len(chunks))
            for off, size in missing:
                # a parameter that received no gradient: zeros, as the zeroed
                # grad buffer of the reference gives it (layer_state.py:297);
                # no copy writes these ranges
                rt.grad_ring.slots[slot][off:off + size].zero_()
            master_before = self._cpu_params_flat.clone() if rt.capture is not None else None
            staging = self._open_staging_pieces(plan[0]) if plan is not None and rt.stage_after_update else None
            try:
                rt.set_adam_threads()
                with self.update_lock:
                    if self.layer_optimizer is not None:
                        # The fp32 masters are passed explicitly: this thread
                        # never reads param.data, which the autograd thread may
                        # be rebinding at the same time.
                        self.layer_optimizer.step_with_grad_views(
                            self.layer_idx, self._grad_views(rt.grad_ring.slots[slot]),
                            param_views=self._master_views(), bf16_views=self._bf16_views(),
                            pieces=None if plan is None else plan[1],
                            before_piece=None if plan is None else wait_chunks,
                            after_piece=None if staging is None else staging[1].push)
            except BaseException:
                if staging is not None:
                    staging[1].abort()
                raise
            rt.mark("adam_done", self.layer_idx)
            if staging is not None:
                self._set_prefetched(staging[0], staging[1].close(cast_later=rt.cast_at_use))
                rt.mark("staged_after_update", self.layer_idx)
            elif rt.stage_after_update:
                self.stage_for_next_forward()
            if master_before is not None:
                wait_chunks(len(chunks))
                rt.capture[self.layer_idx] = (rt.grad_ring.slots[slot][:self.total_size].clone(), master_before)
        finally:
            try:
                # every gradient copy has landed before the slot is handed back
                wait_chunks(len(chunks))
                del keep
                if rt.d2h_timing is not None and state["t0"] is not None:
                    rt.d2h_timing.append(("interval_ns", state["t0"], state["t1"], nbytes))
                rt.grad_ring.release(slot)
            finally:
                self.update_finished.set()
        return True

    def update_params(self) -> None:
        """Kept for API compatibility: the update is queued by the offload
        task as soon as the gradients' D2H is issued."""

    def wait_for_update(self, timeout: Optional[float] = None) -> None:
        """Block until this unit's last update finished; re-raise its error.
        A unit whose offload is still queued is waited for as well."""
        t = timeout if timeout is not None else self.runtime.wait_timeout
        if self._d2h_future is not None:
            self._d2h_future.result(timeout=t)
        f = self._update_future
        if f is not None:
            f.result(timeout=t)
        if not self.update_finished.wait(timeout=t):
            raise TimeoutError(f"Layer {self.layer_idx} parameter update timed out")

    def forward(self, *args, **kwargs):
        raise NotImplementedError("LayerRuntimeState manages state; call .layer(...) for compute")
