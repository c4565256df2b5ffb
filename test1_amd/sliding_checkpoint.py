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
  * 16-bit tensors are packed into their slot by a kernel with a capped grid
    instead of the runtime's full-device copy kernel.
  * NVMe/GPUDirect mode (``gds_offload=True``) is not part of this build.
"""

from __future__ import annotations

from collections import deque
from typing import Any, List, Optional, Tuple

import torch
from torch.autograd.graph import saved_tensors_hooks

from . import kernels
from .pinned import pinned_empty

_offload_streams = {}
# Prefetched layers not yet consumed, shared by all SlidingCheckpoint
# instances that have no ActivationRing (the reference's module-level FIFO).
fifo_prefetch_queue: deque = deque()
# Number of tensors packed per (layer_tensors, layer), for instances without a ring.
_packed_counts = {}


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

    def __init__(self, device):
        self.device = torch.device(device)
        self.sets: List[Optional[List[torch.Tensor]]] = [None, None]
        self.next = 0
        self.fifo: deque = deque()
        self.packed_counts = {}

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

    def reset(self) -> None:
        self.fifo.clear()


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
        max_workgroups: int = 8,
        prefetch_stream: Optional[torch.cuda.Stream] = None,
        pack_fence=None,
    ):
        if gds_offload:
            raise NotImplementedError("SlidingCheckpoint: NVMe (GPUDirect Storage) offload is not supported")
        if layer_tensors is None:
            raise ValueError("SlidingCheckpoint: layer_tensors is required for host offload")
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
        self._key = id(layer_tensors)
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
            slots = self.layer_tensors[self.layer_idx]
            while len(slots) <= self.pack_counter:
                slots.append(None)
            slot = slots[self.pack_counter]
            if slot is None or slot.shape != tensor.shape or slot.dtype != tensor.dtype:
                # First use of this slot (the mask slot is created on demand)
                # or a new batch shape: (re)allocate it, pinned and exact-size.
                slot = pinned_empty(tensor.shape, tensor.dtype)
                slots[self.pack_counter] = slot
            cur = torch.cuda.current_stream()
            if self.pack_counter == 0:
                self.pre_pack_event.record(cur)
                self.stream.wait_event(self.pre_pack_event)
                if self.pack_fence is not None:
                    self.pack_fence(self.stream)
                if self._trace is not None:
                    self._trace("act_d2h", self.layer_idx + 1)
            src = tensor.detach()
            if not src.is_contiguous():
                with torch.cuda.stream(self.stream):
                    src = src.contiguous()
            if src.element_size() == 2:
                # 16-bit tensors are packed by a capped-grid kernel writing
                # straight into the pinned slot (a few CUs keep the link busy).
                kernels.copy_segs_b16([(src.view(-1), slot.view(-1))], self.stream,
                                      max_workgroups=self.max_workgroups)
            else:
                kernels.memcpy_async(slot, src, self.stream)
            src.record_stream(self.stream)
            self.pack_counter += 1
            self._counts[(self._key, self.layer_idx)] = self.pack_counter
            return (tensor.device, slot)

        def unpack_hook(packed: Tuple[torch.device, Any]) -> torch.Tensor:
            device, tensor = packed
            if tensor.size() == torch.Size([0]):
                return torch.empty(tensor.shape, dtype=tensor.dtype, device=device)
            if not pin_memory:
                return tensor.to(device, non_blocking=pin_memory)
            cur = torch.cuda.current_stream()
            if self.unpack_counter == 0:
                self.pre_unpack_event.record(cur)
                nxt = self.layer_idx - 1
                if nxt >= 0:
                    host = self.layer_tensors[nxt][: self._slots_used(nxt)]
                    if self.ring is not None:
                        bufs = self.ring.buffers_like(host)
                    else:
                        bufs = [torch.empty(t.shape, dtype=t.dtype, device=self.device) for t in host]
                    ps = self.prefetch_stream
                    ps.wait_event(self.pre_unpack_event)
                    for h, d in zip(host, bufs):
                        kernels.memcpy_async(d, h, ps)
                        if self.ring is None:
                            d.record_stream(ps)
                    ev = torch.cuda.Event()
                    ev.record(ps)
                    self.fifo.append((bufs, ev))
                    if self._trace is not None:
                        self._trace("act_h2d", nxt + 1)
            if self.is_last_layer:
                self.unpack_counter += 1
                return tensor
            if not self.fifo:
                # Nothing was prefetched for this layer (e.g. a first-layer
                # recompute outside the sliding order): synchronous fallback.
                return tensor.to(device, non_blocking=True)
            bufs, ev = self.fifo[0]
            if self.unpack_counter == 0:
                cur.wait_event(ev)
            result = bufs[self.unpack_counter]
            self.unpack_counter += 1
            # Pop once every prefetched tensor of this layer has been served.
            # (The reference pops after the first tensor when no_mask is set,
            # sliding_checkpoint.py:128, which misroutes a layer that saves
            # more than one tensor; the count is exact in both cases.)
            if self.unpack_counter == len(bufs):
                self.fifo.popleft()
            return result

        super().__init__(pack_hook, unpack_hook)

    def _slots_used(self, layer: int) -> int:
        """Number of tensors layer ``layer`` packed in this step's forward."""
        return self._counts.get((self._key, layer), 0)
