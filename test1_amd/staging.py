"""Device side of a unit's weights: the 2-unit pool, the H2D paths and the
pieces a unit's update and staging can be split into.

* ``LayerBufferPool`` (reference layer_state.py:28-101): fixed set of device
  units reused in FIFO order, each with a ``ready`` event its next writer
  waits on.
* ``H2DStager``: pinned fp32 master -> device fp32 (DMA on ``h2d_stream``)
  -> bf16 or fp16 unit (HIP cast kernel), through a ring of chunk slots or a
  whole-unit slot whose cast can wait until the unit is used; replaces the
  host cast + bf16 copy of reference layer_state.py:296-314.
* ``BF16Loader``: the host optimizer's pinned bf16 copy -> device bf16 unit,
  one DMA per unit (the reference's link format without its host cast).
* ``split_into_pieces`` / ``overlap_ranges``: flat ranges of a unit that
  keep the host AdamW's per-element arithmetic of the whole-unit call.
"""

from __future__ import annotations

import bisect
import contextlib
import itertools
import threading
from collections import deque
from typing import Any, Dict, List, Optional, Sequence, Tuple

import torch

from . import kernels


def _new_event() -> torch.cuda.Event:
    return torch.cuda.Event(enable_timing=False, blocking=False)


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
    callers then stage through the ring.

    New buffers are allocated with ``alloc_stream`` (the stream that copies
    into them) current.  The caching allocator hands a stream the blocks last
    freed on it, ordered only with that stream's own work: a buffer taken on
    the compute stream (the update thread's current stream is the same
    default stream) may be memory the backward has freed while its kernels
    on it are still queued, and a copy on another stream would then overwrite
    it under them."""

    def __init__(self, device: torch.device, cap_bytes: int, alloc_stream: Optional[torch.cuda.Stream] = None):
        self.device = device
        self.alloc_stream = alloc_stream
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
                with (torch.cuda.stream(self.alloc_stream) if self.alloc_stream is not None
                      else contextlib.nullcontext()):
                    t = torch.empty(n, dtype=torch.float32, device=self.device)
            except torch.cuda.OutOfMemoryError:
                self.disabled = True
                return None
            self.bytes += 4 * n
            return t, None

    def give(self, t: torch.Tensor, free_event: Optional[torch.cuda.Event]) -> None:
        with self._lock:
            self._free.setdefault(t.numel(), []).append((t, free_event))

    def release(self, timeout: Optional[float] = None) -> None:
        """Drop the free buffers once the work that last read each one has
        completed (its event: a cast, on whatever stream ran it); buffers
        still out stay with their holders.  The caller has drained the copy
        stream.  A dropped buffer goes back to the caching allocator on the
        copy stream, which every runtime of the process shares: the next
        runtime's copy into it would not wait for a cast still queued on
        another stream."""
        with self._lock:
            dropped = [b for lst in self._free.values() for b in lst]
            self._free.clear()
        for t, ev in dropped:
            if ev is not None:
                kernels.wait_event(ev, timeout, "a staging slot's last cast")
        with self._lock:
            self.bytes -= sum(4 * t.numel() for t, _ in dropped)


class H2DStager:
    """Pinned fp32 master -> device bf16 (or fp16) unit, through a device fp32 ring.

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
        self.slots = _SlotPool(device, slot_cap_bytes, alloc_stream=h2d_stream)

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
                kernels.cast_f32_16_(dst_bf16[off:off + c], self._slot(s, c), self.cast_stream, timer=timer)
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
        kernels.cast_f32_16_(dst_bf16[:p.n], p.slot[:p.n], stream, timer=timer)
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
        self.last_issued: Optional[torch.cuda.Event] = None   # the latest piece's copy
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
        self.last_issued = copied
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
        """Give the slot back without casting (the unit is staged whole later).
        Its next writer waits for what this one waited for: the slot's last
        reader when no piece was pushed, else the last piece's copy (issued
        after that reader, on the same stream)."""
        if self.open:
            self.open = False
            self.stager.slots.give(self.buf, self.slot_free if self.pushed == 0 else self.last_issued)


class BF16Loader:
    """Pinned bf16 host copy -> device bf16 unit: one DMA per unit, no cast.

    Used when the host optimizer keeps a bf16 copy of every master current
    (it writes it in the same pass as the update), so two bytes per parameter
    cross the host link -- the reference's link format (layer_state.py:299-314)
    without its host cast on the load path.  Offers the stager's fence
    interface; there are no casts to fence behind.
    """

    def __init__(self, h2d_stream: torch.cuda.Stream, timing_source=None):
        self.h2d_stream = h2d_stream
        self._copies: deque = deque()
        self.last_cast_done: Optional[torch.cuda.Event] = None
        self.cast_timing: Optional[list] = None
        self._copy_timing: Optional[list] = None
        # With a ``timing_source`` (the fp32 stager whose backward reloads
        # this loader takes over), copies are timed in that object's list.
        self._timing_source = timing_source

    @property
    def copy_timing(self) -> Optional[list]:
        src = self._timing_source
        return self._copy_timing if src is None else src.copy_timing

    @copy_timing.setter
    def copy_timing(self, value: Optional[list]) -> None:
        if self._timing_source is None:
            self._copy_timing = value
        else:
            self._timing_source.copy_timing = value

    def fence_after_casts(self, stream: torch.cuda.Stream) -> None:
        return None

    def load(self, host_bf16: torch.Tensor, dst_bf16: torch.Tensor,
             wait_event: Optional[torch.cuda.Event]) -> torch.cuda.Event:
        n = host_bf16.numel()
        if dst_bf16.numel() < n:
            raise ValueError("BF16Loader.load: destination smaller than source")
        if wait_event is not None:
            self.h2d_stream.wait_event(wait_event)
        timing_list = self.copy_timing
        timing = timing_list is not None
        if timing:
            t0 = torch.cuda.Event(enable_timing=True)
            t0.record(self.h2d_stream)
        kernels.memcpy_async(dst_bf16[:n], host_bf16, self.h2d_stream)
        done = torch.cuda.Event(enable_timing=True) if timing else _new_event()
        done.record(self.h2d_stream)
        if timing:
            timing_list.append((t0, done, n * 2))
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
