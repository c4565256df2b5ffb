"""SlidingCheckpoint: offload checkpoint inputs to pinned host slots and
prefetch them back one layer ahead in backward.

Reference sliding_checkpoint.py:11-131 (CPU mode).  The contract is the same
``saved_tensors_hooks`` pair around a non-reentrant ``checkpoint`` call:

* pack (forward): a tensor of shape ``(0,)`` or, with ``pin_memory=False``,
  any tensor goes to the host with ``.cpu()``; the last decoder keeps its GPU
  tensor; every other tensor is copied asynchronously into
  ``layer_tensors[layer][counter]`` on the offload stream after the
  producing stream has reached this point.
* unpack (backward recompute): on the first tensor of layer j, the slots of
  layer j-1 are copied back to the GPU on the offload stream and queued on a
  FIFO; layer j itself is served from the head of that FIFO.

What is different, and why:
  * the copy source is fenced with ``record_stream`` so the caching
    allocator cannot hand its memory out while the D2H still reads it (the
    reference omits this, sliding_checkpoint.py:69-73);
  * the consumer waits for the prefetch with a stream-side ``wait_event``
    instead of blocking the autograd thread (sliding_checkpoint.py:121);
  * prefetch buffers come from a preallocated two-slot device ring
    (``ActivationRing``) when one is given, instead of ``empty_like`` per
    layer;
  * events are recorded on the current stream rather than the null stream;
  * the checkpoint's empty placeholder tensor is not round-tripped through
    blocking copies;
  * with ``pack_engine="sdma"`` each checkpoint goes to its slot on an SDMA
    engine, started by a worker thread once the tensor is produced (a kernel
    writing into host memory slows the kernels beside it); otherwise 16-bit
    tensors are packed into their slot by a kernel with a capped grid instead
    of the runtime's full-device copy kernel.

Storage mode (``gds_offload=True``, reference sliding_checkpoint.py:133-202):
the reference writes each checkpoint input from device memory straight to
``file_paths[layer][counter]`` with kvikio (GPUDirect Storage) and reads layer
j-1 back into a new device buffer when layer j is first unpacked.  This
platform has no GPU-to-storage DMA, so a ``StorageSpill`` stages through a few
pinned bounce slots instead: pack copies the tensor into a slot (on the
offload stream, or on an SDMA engine started by the worker thread), and a
worker thread writes the slot to the file once the copy has landed; the prefetch of layer j-1 waits for that layer's writes, reads
each file into a slot and copies it to the device on the prefetch stream.
The consumer waits for the prefetch on its stream, as in host mode.  Files
are opened through the native storage engine (O_DIRECT where available) and
unlinked at once, so no file outlives the process.
"""

from __future__ import annotations

import threading
import time
from collections import deque
from concurrent.futures import Future, ThreadPoolExecutor
from typing import Any, Dict, List, Optional, Tuple

import torch
from torch.autograd.graph import saved_tensors_hooks
# The reference module also carries a copy of torch's save_on_cpu
# (sliding_checkpoint.py:206-231); torch's own class is the same interface.
from torch.autograd.graph import save_on_cpu  # noqa: F401

from . import _native, kernels, storage
from .pinned import pinned_empty

_offload_streams = {}
# Prefetched layers not yet consumed, shared by all SlidingCheckpoint
# instances that have no ActivationRing (the reference's module-level FIFO).
fifo_prefetch_queue: deque = deque()
# Number of tensors packed per (layer_tensors, layer), for instances without a ring.
_packed_counts = {}
# Storage mode: (path, shape, dtype) of each tensor packed per (file_paths, layer).
_packed_meta = {}


def offload_stream(device) -> torch.cuda.Stream:
    """The activation offload stream of ``device`` (created on first use)."""
    dev = torch.device(device)
    key = dev.index if dev.index is not None else torch.cuda.current_device()
    s = _offload_streams.get(key)
    if s is None:
        s = torch.cuda.Stream(device=torch.device("cuda", key))
        _offload_streams[key] = s
    return s


class ActivationRing:
    """Two device buffer sets for prefetched checkpoint inputs, reused
    alternately, plus the FIFO of prefetched layers.

    The set filled for layer j-1 was last read by layer j+1's recompute and
    backward; its refill is ordered after them because the offload stream
    waits on an event recorded on the compute stream after layer j+1's
    backward has been enqueued."""

    def __init__(self, device, host_lead: int = 2, wait_timeout: Optional[float] = 600.0):
        self.device = torch.device(device)
        self.sets: List[Optional[List[torch.Tensor]]] = [None, None]
        self.next = 0
        self.fifo: deque = deque()
        self.packed_counts = {}
        self.packed_meta = {}
        # The compute-stream events recorded at each layer's first unpack in
        # this backward, most recent last; see ``throttle``.
        self.host_lead = int(host_lead)
        self.unpack_events: deque = deque(maxlen=max(8, self.host_lead))
        self.wait_timeout = wait_timeout
        # Checkpoint copies into pinned slots.  Kernel packs on a stream: per
        # (model key, decoder) an event after that decoder's last pack, which
        # its prefetch waits for.  SDMA packs (``issue_pack``): per (model key,
        # decoder) the copies not yet seen complete, each with the source it
        # reads, which stays referenced until then; the prefetch settles them.
        self.packed_events: Dict[Tuple[int, int], torch.cuda.Event] = {}
        self.pending_packs: Dict[Tuple[int, int], List[Tuple[Future, torch.Tensor, int]]] = {}
        self._packs_lock = threading.Lock()
        self._pack_issuer: Optional[ThreadPoolExecutor] = None
        # Copies that did not complete within the wait limit: their sources
        # and slots are kept for the life of the process.
        self._stuck: List[Any] = []

    def throttle(self, what: str) -> None:
        """Before a prefetch is issued: hold the host until the compute
        stream has reached the first unpack ``host_lead`` layers back (0: no
        hold).  Each prefetch copy waits on the compute stream, and the HIP
        runtime puts a copy on the first SDMA engine not already held, a
        waiting copy holding its engine until its event fires.  With the
        host many layers ahead of the device in the backward, the waiting
        prefetches held up to nine engines at once (Qwen2.5-14B step), and
        the parameter and gradient copies queued behind them.  Measured
        (tokens/s, same box): Qwen2.5-14B 3,939 with no hold, 5,000-5,034
        with a lead of 1 layer, 5,162 with 2, 5,019 with 3; Llama-3.1-8B
        5,591 with no hold, 4,683 with 1 (the host then starves the device
        of queued work), 5,759-5,788 with 2, 5,785 with 3."""
        if self.host_lead <= 0 or len(self.unpack_events) < self.host_lead:
            return
        kernels.wait_event(self.unpack_events[-self.host_lead], self.wait_timeout, what)

    def buffers_like(self, host_tensors: List[torch.Tensor]) -> List[torch.Tensor]:
        i = self.next
        self.next ^= 1
        cur = self.sets[i]
        ok = cur is not None and len(cur) == len(host_tensors) and all(
            a.shape == b.shape and a.dtype == b.dtype for a, b in zip(cur, host_tensors))
        if not ok:
            cur = [torch.empty(t.shape, dtype=t.dtype, device=self.device) for t in host_tensors]
            self.sets[i] = cur
        return cur

    def issue_pack(self, key: int, layer: int, src: torch.Tensor, slot: torch.Tensor,
                   ready: torch.cuda.Event) -> None:
        """Copy the contiguous device tensor ``src`` into the pinned host
        ``slot`` on an SDMA engine once ``ready`` (recorded on the producer's
        stream) has completed.  Returns at once: a worker thread waits for
        ``ready`` and starts the copy.  An SDMA engine needs no compute unit,
        where a kernel writing into host memory slows the kernels beside it
        (a bf16 GEMM of Qwen2.5-14B's MLP shape ran 24-27 % slower beside the
        16-workgroup pack kernel, unchanged beside an SDMA copy)."""
        if self._pack_issuer is None:
            self._pack_issuer = ThreadPoolExecutor(max_workers=1, thread_name_prefix="sf-ckpt-d2h")
        timeout = self.wait_timeout

        def task():
            kernels.wait_event(ready, timeout, f"decoder {layer}: checkpoint before its copy to the host")
            return kernels.DmaReady(kernels.dma_copy_d2h([(src.reshape(-1), slot.reshape(-1))], timeout=timeout),
                                    timeout=timeout)

        nbytes = src.numel() * src.element_size()
        fut = self._pack_issuer.submit(task)
        with self._packs_lock:
            self.pending_packs.setdefault((key, layer), []).append((fut, src, nbytes))

    def settle_packs(self, key: int, layer: int, timing: Optional[list] = None) -> None:
        """Wait until the SDMA copies of ``layer``'s checkpoints have landed
        (bounded by the wait limit) and release them and their sources.
        ``timing`` receives ("interval_ns", start, end, bytes) per copy, or
        ("untimed", bytes) without engine timestamps."""
        with self._packs_lock:
            pending = self.pending_packs.pop((key, layer), [])
        for i, (fut, src, nbytes) in enumerate(pending):
            try:
                ready = fut.result(timeout=self.wait_timeout)
                ready.synchronize()
            except BaseException:
                # a copy may still be running (or was never started): keep
                # every source of this layer referenced for good
                self._stuck.append(pending[i:])
                raise
            t0, t1 = ready.release()
            if timing is not None:
                timing.append(("interval_ns", t0, t1, nbytes) if t1 > t0 else ("untimed", nbytes))

    def drain_packs(self) -> None:
        """``settle_packs`` for every layer with copies pending."""
        with self._packs_lock:
            keys = list(self.pending_packs)
        for key, layer in keys:
            self.settle_packs(key, layer)

    def close(self) -> None:
        """Settle every pending copy and stop the worker thread."""
        self.drain_packs()
        if self._pack_issuer is not None:
            self._pack_issuer.shutdown(wait=True)
            self._pack_issuer = None

    def reset(self) -> None:
        self.drain_packs()
        self.packed_events.clear()
        self.fifo.clear()
        self.unpack_events.clear()


class KeptOnDevice:
    """A checkpoint slot that could not be pinned (the driver's pinned-memory
    limit): that checkpoint stays in device memory, as the last decoder's
    does, and its layer's prefetch has nothing to copy for it."""

    __slots__ = ("shape", "dtype")

    def __init__(self, shape, dtype):
        self.shape, self.dtype = torch.Size(shape), dtype


def pin_or_keep(shape, dtype):
    """A pinned slot of ``shape``/``dtype``, or ``KeptOnDevice`` when the
    host cannot pin it."""
    try:
        return pinned_empty(shape, dtype)
    except _native.NativeError as e:
        if e.status != _native.HIP_ERROR_OUT_OF_MEMORY:
            raise
        return KeptOnDevice(shape, dtype)


class _OnStorage:
    """What pack returns for a tensor written to storage."""

    __slots__ = ("path", "shape", "dtype")

    def __init__(self, path: str, shape, dtype):
        self.path, self.shape, self.dtype = path, shape, dtype


class _Unless:
    """A waitable that is complete while ``flags`` is empty."""

    __slots__ = ("flags",)

    def __init__(self, flags: List[Any]):
        self.flags = flags

    def query(self) -> bool:
        return not self.flags


class _BounceSlot:
    __slots__ = ("buf", "held", "pending")

    def __init__(self, nbytes: int):
        self.buf = pinned_empty((storage.align_up(nbytes),), torch.uint8)
        if self.buf.data_ptr() % storage.ALIGN:
            raise RuntimeError("StorageSpill: pinned slot not aligned for direct I/O")
        self.held = False
        self.pending: List[Any] = []   # waitables that must finish before reuse

    def idle(self) -> bool:
        for w in self.pending:
            if isinstance(w, Future):
                if not w.done() or (w.exception() is None and not w.result().done()):
                    return False
            elif not w.query():
                return False
        self.pending = []
        return True


class StorageSpill:
    """Checkpoint inputs on local storage: pinned bounce slots, one file per
    (layer, tensor) path, and one worker thread that turns finished device
    copies into file writes and file reads into device copies (storage mode
    of ``SlidingCheckpoint``)."""

    def __init__(self, n_slots: int = 4, engine: Optional[storage.IoEngine] = None, direct: bool = True):
        if n_slots < 2:
            raise ValueError("StorageSpill: at least 2 bounce slots")
        self.engine = engine or storage.default_engine()
        self.direct = direct
        self.n_slots = n_slots
        self._slots: List[_BounceSlot] = []
        self._files: Dict[str, storage.OffloadFile] = {}
        self._writes: Dict[str, Future] = {}
        self._lock = threading.Lock()
        self._worker = ThreadPoolExecutor(max_workers=1, thread_name_prefix="act-spill")
        self.bytes_written = 0
        self.bytes_read = 0
        self.slot_wait_s = 0.0

    def _file(self, path: str) -> storage.OffloadFile:
        with self._lock:
            f = self._files.get(path)
            if f is None:
                f = self.engine.open(path, direct=self.direct, unlink=True)
                self._files[path] = f
            return f

    def take_slot(self, nbytes: int) -> _BounceSlot:
        """A bounce slot of at least ``nbytes``, waiting for one to drain."""
        t0 = time.perf_counter()
        while True:
            with self._lock:
                for sl in self._slots:
                    if not sl.held and sl.idle():
                        if sl.buf.numel() < nbytes:
                            sl.buf = _BounceSlot(nbytes).buf
                        sl.held = True
                        break
                else:
                    sl = None
                    if len(self._slots) < self.n_slots:
                        sl = _BounceSlot(nbytes)
                        sl.held = True
                        self._slots.append(sl)
            if sl is not None:
                self.slot_wait_s += time.perf_counter() - t0
                return sl
            time.sleep(200e-6)

    def write_after(self, path: str, slot: _BounceSlot, copied: torch.cuda.Event, nbytes: int) -> None:
        """Write ``nbytes`` of ``slot`` to ``path`` once ``copied`` (the
        device-to-slot copy) has completed; the slot is free after the write."""
        f = self._file(path)
        padded = storage.align_up(nbytes)

        def task():
            copied.synchronize()
            return f.write(slot.buf, 0, padded)

        fut = self._worker.submit(task)
        with self._lock:
            self._writes[path] = fut
            slot.pending = [fut]
            slot.held = False
        self.bytes_written += padded

    def write_after_dma(self, path: str, slot: _BounceSlot, src: torch.Tensor, ready: torch.cuda.Event,
                        nbytes: int, timeout: Optional[float], timing: Optional[list] = None) -> None:
        """Copy the contiguous device tensor ``src`` (``nbytes``) into ``slot``
        on an SDMA engine once ``ready`` (recorded after its producer) has
        completed, then write it to ``path``; all on the worker thread, which
        keeps ``src`` referenced until the copy has landed.  ``timing``
        receives the copy's ("interval_ns", start, end, bytes), or
        ("untimed", bytes) without engine timestamps.  A copy that does not
        complete within ``timeout`` keeps the slot and ``src`` for good."""
        f = self._file(path)
        padded = storage.align_up(nbytes)
        stuck: List[Any] = []

        def task():
            kernels.wait_event(ready, timeout, f"checkpoint {path}: before its copy to the host")
            dma = kernels.DmaReady(kernels.dma_copy_d2h([(src.reshape(-1), slot.buf[:nbytes])], timeout=timeout),
                                   timeout=timeout)
            try:
                t0, t1 = dma.release()
            except BaseException:
                stuck.append((dma, src))
                raise
            if timing is not None:
                timing.append(("interval_ns", t0, t1, nbytes) if t1 > t0 else ("untimed", nbytes))
            return f.write(slot.buf, 0, padded)

        fut = self._worker.submit(task)
        with self._lock:
            self._writes[path] = fut
            # never idle again if the copy is stuck
            slot.pending = [fut, _Unless(stuck)]
            slot.held = False
        self.bytes_written += padded

    def prefetch(self, items: List[Tuple[str, torch.Tensor]], after: torch.cuda.Event,
                 stream: torch.cuda.Stream) -> Future:
        """Read each ``(path, device_buffer)`` back into its buffer: on the
        worker, wait for the file's write, read it into a slot, then copy the
        slot to the buffer on ``stream`` after ``after``.  The future gives
        the event recorded after the last copy."""

        def task():
            with torch.cuda.device(stream.device):
                return copy_back()

        def copy_back():
            ev = None
            for path, dst in items:
                nbytes = dst.numel() * dst.element_size()
                padded = storage.align_up(nbytes)
                w = self._writes.get(path)
                if w is None:
                    raise RuntimeError(f"StorageSpill: {path} was never written")
                w.result().wait()
                slot = self.take_slot(padded)
                try:
                    self._file(path).read(slot.buf, 0, padded).wait()
                    stream.wait_event(after)
                    kernels.memcpy_async(dst.view(-1).view(torch.uint8), slot.buf, stream, nbytes=nbytes)
                    ev = torch.cuda.Event()
                    ev.record(stream)
                finally:
                    with self._lock:
                        if ev is not None:
                            slot.pending = [ev]
                        slot.held = False
                self.bytes_read += padded
            return ev

        return self._worker.submit(task)

    def flush(self) -> None:
        """Wait for every queued write (re-raising its error)."""
        for fut in list(self._writes.values()):
            fut.result().wait()

    def close(self) -> None:
        self.flush()
        self._worker.shutdown(wait=True)
        for f in self._files.values():
            f.close()
        self._files.clear()
        self._slots.clear()


_default_spill: Optional[StorageSpill] = None


def default_spill() -> StorageSpill:
    """The process's spill for ``SlidingCheckpoint``s given none (the
    reference keeps its storage-mode state in module globals too)."""
    global _default_spill
    if _default_spill is None:
        _default_spill = StorageSpill()
    return _default_spill


class SlidingCheckpoint(saved_tensors_hooks):
    """Reference signature (sliding_checkpoint.py:13-24) plus ``prefetch_ring``."""

    def __init__(
        self,
        layer_idx: int,
        layer_tensors: Optional[List[List[torch.Tensor]]] = None,
        gds_offload: bool = False,
        file_paths=None,
        is_last_layer: bool = False,
        no_mask: bool = False,
        device: str = "cuda:0",
        pin_memory: bool = True,
        stream: Optional[torch.cuda.Stream] = None,
        prefetch_ring: Optional[ActivationRing] = None,
        trace=None,
        max_workgroups: int = 16,
        prefetch_stream: Optional[torch.cuda.Stream] = None,
        pack_fence=None,
        spill: Optional[StorageSpill] = None,
        link_timing: Optional[dict] = None,
        on_prefetch_ready=None,
        before_pin=None,
        served=None,
        pack_engine: str = "kernel",
    ):
        if pack_engine not in ("kernel", "sdma"):
            raise ValueError("SlidingCheckpoint: pack_engine must be 'kernel' or 'sdma'")
        if gds_offload:
            if file_paths is None:
                raise ValueError("SlidingCheckpoint: file_paths is required for storage offload")
            self.spill = spill or default_spill()
        elif layer_tensors is None:
            raise ValueError("SlidingCheckpoint: layer_tensors is required for host offload")
        self.gds_offload = gds_offload
        self.file_paths = file_paths
        self.layer_idx = layer_idx - 1  # decoder index; units count the embedding as 0
        self.device = device
        self.stream = stream or offload_stream(device)
        # Stream of the backward prefetch (host -> device); the offload stream
        # unless given.  SlideFSDP puts the prefetch on its parameter H2D
        # stream, in FIFO order behind the parameter load of the same layer.
        self.prefetch_stream = prefetch_stream or self.stream
        self.is_last_layer = is_last_layer
        self.no_mask = no_mask
        self.layer_tensors = layer_tensors
        self.ring = prefetch_ring
        self.fifo = prefetch_ring.fifo if prefetch_ring is not None else fifo_prefetch_queue
        self._counts = prefetch_ring.packed_counts if prefetch_ring is not None else _packed_counts
        self._meta = prefetch_ring.packed_meta if prefetch_ring is not None else _packed_meta
        self._key = id(file_paths) if gds_offload else id(layer_tensors)
        self.pack_counter = 0
        self.unpack_counter = 0
        self.pre_pack_event = torch.cuda.Event()
        self.pre_unpack_event = torch.cuda.Event()
        self.post_unpack_event_prefetch = torch.cuda.Event()
        self._trace = trace
        self.max_workgroups = max_workgroups
        # Optional callable(stream): orders the host-writing pack behind other
        # work (SlideFSDP passes its stager's cast fence).
        self.pack_fence = pack_fence
        # Optional measurement: (start, end, bytes) timing events of each pack
        # ("act_d2h") and prefetch ("act_h2d") appended to these lists, and a
        # callable run once the compute stream has been made to wait for this
        # layer's prefetched checkpoint (the recompute starts after it).
        self.link_timing = link_timing
        self.on_prefetch_ready = on_prefetch_ready
        # Optional callable run before a pinned slot is allocated inside the
        # forward (the first step, or a new batch shape): SlideFSDP drains its
        # copies there, since pinning host memory near the driver's limit
        # while copies into pinned memory ran has left wrong results.
        self.before_pin = before_pin
        # Optional dict: (decoder index, tensor index) -> a device copy of each
        # checkpoint tensor the recompute is given, taken on its stream after
        # the prefetch wait (what the recompute reads); for checking only.
        self.served = served
        # How a checkpoint reaches its pinned slot (or, on storage, its bounce
        # slot): "kernel", a capped-grid kernel on ``stream``; "sdma", an SDMA
        # engine (``ActivationRing.issue_pack``, ``StorageSpill.
        # write_after_dma``; needs ``prefetch_ring`` and a contiguous tensor,
        # else the kernel is used).
        self.pack_engine = pack_engine

        def pack_hook(tensor: torch.Tensor) -> Tuple[torch.device, Any]:
            if tensor.size() == torch.Size([0]):
                # The checkpoint's empty placeholder: nothing to copy.  The
                # reference's `.cpu()` (sliding_checkpoint.py:54-55) is a
                # blocking copy that stalls the host on every layer.
                return (tensor.device, torch.empty(tensor.shape, dtype=tensor.dtype))
            if not pin_memory:
                return (tensor.device, tensor.cpu())
            if self.is_last_layer:
                return (tensor.device, tensor)
            nbytes = tensor.numel() * tensor.element_size()
            if self.gds_offload:
                bounce = self.spill.take_slot(nbytes)
                slot = bounce.buf[:nbytes].view(tensor.dtype).view(tensor.shape)
            else:
                slots = self.layer_tensors[self.layer_idx]
                while len(slots) <= self.pack_counter:
                    slots.append(None)
                slot = slots[self.pack_counter]
                if slot is None or slot.shape != tensor.shape or slot.dtype != tensor.dtype:
                    # First use of this slot (the mask slot is created on demand)
                    # or a new batch shape: (re)allocate it, pinned and exact-size.
                    if self.before_pin is not None:
                        self.before_pin()
                    slot = pin_or_keep(tensor.shape, tensor.dtype)
                    slots[self.pack_counter] = slot
            cur = torch.cuda.current_stream()
            if self.pack_counter == 0:
                self.pre_pack_event.record(cur)
                self.stream.wait_event(self.pre_pack_event)
                if self.pack_fence is not None:
                    self.pack_fence(self.stream)
                if self._trace is not None:
                    self._trace("act_d2h", self.layer_idx + 1)
            if isinstance(slot, KeptOnDevice):
                # no pinned slot: the checkpoint stays in device memory
                self.pack_counter += 1
                self._counts[(self._key, self.layer_idx)] = self.pack_counter
                return (tensor.device, tensor)
            src = tensor.detach()
            if self.pack_engine == "sdma" and self.ring is not None and src.is_contiguous():
                # an SDMA engine copies it once the compute stream has produced it
                ready = torch.cuda.Event()
                ready.record(cur)
                self.pack_counter += 1
                self._counts[(self._key, self.layer_idx)] = self.pack_counter
                if not self.gds_offload:
                    self.ring.issue_pack(self._key, self.layer_idx, src, slot, ready)
                    return (tensor.device, slot)
                path = self.file_paths[self.layer_idx][self.pack_counter - 1]
                self.spill.write_after_dma(path, bounce, src, ready, nbytes, self.ring.wait_timeout,
                                           None if self.link_timing is None else self.link_timing["act_d2h"])
                return (tensor.device, self._on_storage(path, tensor))
            if not src.is_contiguous():
                with torch.cuda.stream(self.stream):
                    src = src.contiguous()
            t_pack = None
            if self.link_timing is not None:
                t_pack = torch.cuda.Event(enable_timing=True)
                t_pack.record(self.stream)
            if src.element_size() == 2:
                # 16-bit tensors are packed by a capped-grid kernel writing
                # straight into the pinned slot (a few CUs keep the link busy).
                kernels.copy_segs_b16([(src.view(-1), slot.view(-1))], self.stream,
                                      max_workgroups=self.max_workgroups)
            else:
                kernels.memcpy_async(slot, src, self.stream)
            src.record_stream(self.stream)
            if self.ring is not None and not self.gds_offload:
                # this decoder's prefetch waits for its last pack
                packed = torch.cuda.Event()
                packed.record(self.stream)
                self.ring.packed_events[(self._key, self.layer_idx)] = packed
            if t_pack is not None:
                done = torch.cuda.Event(enable_timing=True)
                done.record(self.stream)
                self.link_timing["act_d2h"].append((t_pack, done, nbytes))
            self.pack_counter += 1
            self._counts[(self._key, self.layer_idx)] = self.pack_counter
            if self.gds_offload:
                path = self.file_paths[self.layer_idx][self.pack_counter - 1]
                copied = torch.cuda.Event()
                copied.record(self.stream)
                self.spill.write_after(path, bounce, copied, nbytes)
                return (tensor.device, self._on_storage(path, tensor))
            return (tensor.device, slot)

        def unpack_hook(packed: Tuple[torch.device, Any]) -> torch.Tensor:
            device, tensor = packed
            if isinstance(tensor, torch.Tensor) and tensor.size() == torch.Size([0]):
                return torch.empty(tensor.shape, dtype=tensor.dtype, device=device)
            if not pin_memory:
                return tensor.to(device, non_blocking=pin_memory)
            cur = torch.cuda.current_stream()
            if self.unpack_counter == 0:
                self.pre_unpack_event.record(cur)
                nxt = self.layer_idx - 1
                if nxt >= 0 and self.gds_offload:
                    meta = self._meta.get((self._key, nxt), [])[: self._slots_used(nxt)]
                    if meta:
                        like = [torch.empty(shape, dtype=dt, device="meta") for _, shape, dt in meta]
                        if self.ring is not None:
                            bufs = self.ring.buffers_like(like)
                            self.ring.throttle(f"decoder {self.layer_idx}: the backward before its checkpoint "
                                               f"prefetch")
                            self.ring.unpack_events.append(self.pre_unpack_event)
                        else:
                            bufs = [torch.empty(shape, dtype=dt, device=self.device) for _, shape, dt in meta]
                        ps = self.prefetch_stream
                        fut = self.spill.prefetch([(path, b) for (path, _, _), b in zip(meta, bufs)],
                                                  self.pre_unpack_event, ps)
                        if self.ring is None:
                            for b in bufs:
                                b.record_stream(ps)
                        self.fifo.append((bufs, fut))
                        if self._trace is not None:
                            self._trace("act_h2d", nxt + 1)
                elif nxt >= 0:
                    host = self.layer_tensors[nxt][: self._slots_used(nxt)]
                    # tensors kept in device memory (KeptOnDevice) get no
                    # buffer: their entry is None and the packed tensor is served
                    pinned = [h for h in host if not isinstance(h, KeptOnDevice)]
                    if self.ring is not None:
                        got = self.ring.buffers_like(pinned)
                    else:
                        got = [torch.empty(t.shape, dtype=t.dtype, device=self.device) for t in pinned]
                    it = iter(got)
                    bufs = [None if isinstance(h, KeptOnDevice) else next(it) for h in host]
                    ps = self.prefetch_stream
                    if self.ring is not None:
                        self.ring.throttle(f"decoder {self.layer_idx}: the backward before its checkpoint "
                                           f"prefetch")
                        self.ring.unpack_events.append(self.pre_unpack_event)
                        # the slots are read only after the copies into them
                        self.ring.settle_packs(self._key, nxt,
                                               None if self.link_timing is None else self.link_timing["act_d2h"])
                        packed = self.ring.packed_events.pop((self._key, nxt), None)
                        if packed is not None:
                            ps.wait_event(packed)
                    ps.wait_event(self.pre_unpack_event)
                    timed = self.link_timing is not None
                    if timed:
                        t0 = torch.cuda.Event(enable_timing=True)
                        t0.record(ps)
                    for h, d in zip(host, bufs):
                        if d is None:
                            continue
                        kernels.memcpy_async(d, h, ps)
                        if self.ring is None:
                            d.record_stream(ps)
                    ev = torch.cuda.Event(enable_timing=timed)
                    ev.record(ps)
                    if timed:
                        self.link_timing["act_h2d"].append(
                            (t0, ev, sum(h.numel() * h.element_size() for h in pinned)))
                    self.fifo.append((bufs, ev))
                    if self._trace is not None:
                        self._trace("act_h2d", nxt + 1)
            if self.is_last_layer:
                self._record_served(tensor)
                self.unpack_counter += 1
                return tensor
            if not self.fifo:
                # Nothing was prefetched for this layer (e.g. a first-layer
                # recompute outside the sliding order): synchronous fallback.
                if isinstance(tensor, _OnStorage):
                    raise RuntimeError("SlidingCheckpoint: a layer on storage was not prefetched")
                return tensor.to(device, non_blocking=True)
            bufs, ev = self.fifo[0]
            if self.unpack_counter == 0:
                if isinstance(ev, Future):
                    ev = ev.result()
                cur.wait_event(ev)
                if self.on_prefetch_ready is not None:
                    self.on_prefetch_ready()
            result = bufs[self.unpack_counter]
            if result is None:
                result = tensor   # kept in device memory by the pack hook
            self._record_served(result)
            self.unpack_counter += 1
            # Pop once every prefetched tensor of this layer has been served.
            # (The reference pops after the first tensor when no_mask is set,
            # sliding_checkpoint.py:128, which misroutes a layer that saves
            # more than one tensor; the count is exact in both cases.)
            if self.unpack_counter == len(bufs):
                self.fifo.popleft()
            return result

        super().__init__(pack_hook, unpack_hook)

    def _on_storage(self, path: str, tensor: torch.Tensor) -> _OnStorage:
        """Record that this layer's current pack went to ``path``."""
        meta = self._meta.setdefault((self._key, self.layer_idx), [])
        del meta[self.pack_counter - 1:]
        meta.append((path, tuple(tensor.shape), tensor.dtype))
        return _OnStorage(path, tuple(tensor.shape), tensor.dtype)

    def _record_served(self, t: torch.Tensor) -> None:
        if self.served is not None:
            self.served[(self.layer_idx, self.unpack_counter)] = t.detach().clone()

    def _slots_used(self, layer: int) -> int:
        """Number of tensors layer ``layer`` packed in this step's forward."""
        return self._counts.get((self._key, layer), 0)
