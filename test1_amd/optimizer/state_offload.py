"""Optimizer moments on local storage, for LayerAdam's NVMe offload.

Reference: optimizer/layer_adam/layer_adam.py:89-103 (tensornvme
``DiskOffloader``), 186-244 (``_load_layer`` / ``_offload_layer`` /
``_pre_step`` / ``_post_step``).  There, each unit's ``exp_avg`` (and
``exp_avg_sq`` when ``nvme_offload_fraction > 0.5``) is written to a file
after the unit's step and its host memory freed; the step of unit i reads
unit i-1 back ahead of time (updates run in descending unit order).

Here the moments of every unit live in one file (``offload-<pid>-<n>.bin``
in the offload directory, unlinked at once so that the space is returned at
exit), each (unit, moment) in its own 4 KiB-aligned region.  Host memory is a
few buffers, each able to hold the moments of the largest unit:

* ``prefetch(unit, priority)`` requests a unit; reads of requested units
  start, lowest priority first, whenever a buffer can be taken without
  waiting, and a buffer holding a requested unit is kept for it;
* ``acquire(unit)`` returns the unit's moments, waiting for (or starting)
  the read, and for a write-back of the same buffer still in flight;
* ``release(unit)`` queues the write-back of the updated moments.

A buffer keeps its unit's moments after the write-back, so a unit updated
again before its buffer is reused is not read back (its buffer already holds
what the file holds).  Buffers are taken in this order: never used, clean
(written back) and not requested, least recently used first, then -- only
when the caller must wait -- one holding the requested unit needed last (it
is read again later), then the oldest write-back.  Moments reach the optimizer unchanged, so the updates are
those of moments kept in memory, bit for bit.

Unwritten file ranges read as zeros: the initial moments need no writes.
"""

from __future__ import annotations

import itertools
import os
import threading
import time
from typing import Dict, List, Optional, Tuple

import torch

from .. import storage


class _Buffer:
    __slots__ = ("tensors", "capacity", "owner", "reads", "writes", "in_use", "last")

    def __init__(self, kinds: int, numel: int):
        self.tensors = [storage.aligned_empty(numel, torch.float32) for _ in range(kinds)]
        self.capacity = numel
        self.owner: Optional[int] = None
        self.reads: List[storage.IoRequest] = []
        self.writes: List[storage.IoRequest] = []
        self.in_use = False
        self.last = 0

    def grow(self, numel: int) -> None:
        if numel > self.capacity:
            self.tensors = [storage.aligned_empty(numel, torch.float32) for _ in self.tensors]
            self.capacity = numel


class StateOffloader:
    """Moments of the units of one optimizer on a file (see module doc)."""

    _ids = itertools.count()

    def __init__(self, offload_dir: str, n_moments: int, n_buffers: int = 4,
                 engine: Optional[storage.IoEngine] = None, direct: bool = True):
        if n_moments not in (1, 2):
            raise ValueError("StateOffloader: 1 (exp_avg) or 2 (exp_avg, exp_avg_sq) moments")
        if n_buffers < 2:
            raise ValueError("StateOffloader: at least 2 buffers")
        os.makedirs(offload_dir, exist_ok=True)
        self.engine = engine or storage.default_engine()
        path = os.path.join(offload_dir, f"offload-{os.getpid()}-{next(StateOffloader._ids)}.bin")
        self.file = self.engine.open(path, direct=direct, unlink=True)
        self.n_moments = n_moments
        self.n_buffers = n_buffers
        self._layout: Dict[int, Tuple[int, int, List[int]]] = {}  # unit -> (numel, nbytes, offsets)
        self._end = 0
        self._max_numel = 0
        self._buffers: List[_Buffer] = []
        self._where: Dict[int, _Buffer] = {}
        self._requested: Dict[int, Tuple[float, int]] = {}
        self._seq = itertools.count()
        self._tick = itertools.count(1)
        self._lock = threading.RLock()
        self.wait_s = 0.0  # time acquire() spent waiting for reads / write-backs

    # ------------------------------------------------------------------
    def register(self, unit: int, numel: int) -> None:
        """Give ``unit`` (``numel`` fp32 per moment) its file regions."""
        with self._lock:
            if unit in self._layout:
                raise ValueError(f"StateOffloader: unit {unit} registered twice")
            nbytes = storage.align_up(4 * numel)
            offs = [self._end + k * nbytes for k in range(self.n_moments)]
            self._end += self.n_moments * nbytes
            self.file.reserve(self._end)
            self._layout[unit] = (numel, nbytes, offs)
            self._max_numel = max(self._max_numel, numel)

    def units(self) -> List[int]:
        return list(self._layout)

    @property
    def file_bytes(self) -> int:
        return self._end

    @property
    def buffer_bytes(self) -> int:
        return sum(4 * b.capacity * self.n_moments for b in self._buffers)

    # ------------------------------------------------------------------
    # Buffer states: unused (no owner); loading (reads in flight); holding a
    # unit's moments, clean or with its write-back in flight; in use between
    # acquire and release.  A unit is "requested" from prefetch() until its
    # acquire(); a buffer holding a requested unit is protected: reads for
    # other units never take it (only an acquire that must wait may).
    def _reap(self, b: _Buffer) -> None:
        """Release finished write-backs of ``b`` (its contents stay valid)."""
        if b.writes and all(r.done() for r in b.writes):
            b.writes = []

    def _protected(self, b: _Buffer) -> bool:
        return b.owner is not None and b.owner in self._requested

    def _evict(self, b: _Buffer) -> None:
        if b.owner is not None:
            del self._where[b.owner]
        b.owner = None

    def _take(self, blocking: bool) -> Optional[_Buffer]:
        """A buffer for a new unit (under the lock), or None if ``blocking``
        is false and every buffer is busy or protected."""
        for b in self._buffers:
            if not b.in_use and b.owner is None and not b.reads and not b.writes:
                return b
        if len(self._buffers) < self.n_buffers:
            b = _Buffer(self.n_moments, self._max_numel)
            self._buffers.append(b)
            return b
        for b in self._buffers:
            if not b.in_use:
                self._reap(b)
        clean = [b for b in self._buffers
                 if not b.in_use and not b.reads and not b.writes and not self._protected(b)]
        if clean:
            b = min(clean, key=lambda b: b.last)
            self._evict(b)
            return b
        if not blocking:
            return None
        prot = [b for b in self._buffers if not b.in_use and self._protected(b)]
        if prot:
            # the requested unit needed last stays requested and is read again later
            b = max(prot, key=lambda b: self._requested[b.owner])
        else:
            writing = [b for b in self._buffers if not b.in_use and b.writes]
            if not writing:
                raise RuntimeError("StateOffloader: every buffer is in use")
            b = min(writing, key=lambda b: b.last)
        for r in b.reads + b.writes:
            r.wait()
        b.reads, b.writes = [], []
        self._evict(b)
        return b

    def _start_read(self, unit: int, b: _Buffer) -> None:
        numel, nbytes, offs = self._layout[unit]
        b.grow(numel)
        b.owner = unit
        self._where[unit] = b
        b.reads = [self.file.read(t, off, nbytes) for t, off in zip(b.tensors, offs)]

    def _pump(self) -> None:
        """Start reads of requested units, lowest priority first, while
        buffers can be taken without waiting."""
        pending = sorted((key, u) for u, key in self._requested.items() if u not in self._where)
        for _, unit in pending:
            b = self._take(blocking=False)
            if b is None:
                return
            self._start_read(unit, b)

    # ------------------------------------------------------------------
    def prefetch(self, unit: int, priority: float = 0.0) -> None:
        """Request ``unit``'s moments ahead of its update (lower priority
        first); they stay requested until ``acquire``."""
        with self._lock:
            if unit not in self._layout:
                return
            if unit not in self._requested:
                self._requested[unit] = (priority, next(self._seq))
            self._pump()

    def ready(self, unit: int) -> bool:
        """True if ``acquire(unit)`` would not wait: its moments are in a
        buffer with no transfer in flight."""
        with self._lock:
            b = self._where.get(unit)
            if b is None:
                self._pump()
                return False
            return all(r.done() for r in b.reads + b.writes)

    def acquire(self, unit: int) -> List[torch.Tensor]:
        """The moments of ``unit`` (fp32 views of ``numel`` elements), to be
        updated in place and handed back with ``release``."""
        t0 = time.perf_counter()
        with self._lock:
            numel = self._layout[unit][0]
            self._requested.pop(unit, None)
            b = self._where.get(unit)
            if b is None:
                b = self._take(blocking=True)
                self._start_read(unit, b)
            if b.in_use:
                raise RuntimeError(f"StateOffloader: unit {unit} acquired twice")
            b.in_use = True
            pending = b.reads + b.writes
        # Wait outside the lock (the buffer is in use, so nobody takes it);
        # keep other reads going while this one completes.
        for r in pending:
            while not r.done():
                with self._lock:
                    self._pump()
                time.sleep(200e-6)
        with self._lock:
            b.reads = []
            b.writes = []
        self.wait_s += time.perf_counter() - t0
        return [t[:numel] for t in b.tensors]

    def release(self, unit: int, dirty: bool = True) -> None:
        """Hand back ``unit``'s moments; ``dirty`` queues their write-back."""
        with self._lock:
            b = self._where[unit]
            if not b.in_use:
                raise RuntimeError(f"StateOffloader: unit {unit} released but not acquired")
            if dirty:
                _, nbytes, offs = self._layout[unit]
                b.writes = [self.file.write(t, off, nbytes) for t, off in zip(b.tensors, offs)]
            b.in_use = False
            b.last = next(self._tick)
            self._pump()

    def read_back(self, unit: int) -> List[torch.Tensor]:
        """Copies of ``unit``'s current moments."""
        views = self.acquire(unit)
        try:
            return [v.clone() for v in views]
        finally:
            self.release(unit, dirty=False)

    def flush(self) -> None:
        """Wait for every queued transfer."""
        with self._lock:
            reqs = [r for b in self._buffers for r in b.reads + b.writes]
        for r in reqs:
            r.wait()
        with self._lock:
            for b in self._buffers:
                if not b.in_use:
                    b.writes = []
                    # reads of prefetched buffers stay listed: acquire clears them

    def close(self) -> None:
        self.flush()
        self.file.close()
        self._buffers = []
        self._where = {}
