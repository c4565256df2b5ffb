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

This module holds the objects shared by all units (``StreamingRuntime``) and
the runtime of one unit (``LayerRuntimeState``).  The pool and the H2D paths
are in ``staging``, the pinned gradient slots in ``grad_slots``, the worker
threads in ``update_executor`` and the row-sparse embedding in
``embedding_rows``; the names the reference's layer_state module exports
(``LayerBufferPool``, ``LayerRuntimeState``) are importable from here.

Memory layout in HBM (per unit, offset-identical to the fp32 master):
  unit["param"]  bf16 weights (pool units: ``max_param_size`` elements)
plus the fp32 staging ring (``depth`` chunks of ``chunk_elems``) with fp32 H2D.
"""

from __future__ import annotations

import threading
import time
from collections import OrderedDict
from concurrent import futures
from concurrent.futures import Future
from typing import Any, Callable, Dict, List, Optional, Tuple

import torch
import torch.nn as nn

from . import _native, kernels
from .embedding_rows import RowSparseEmbedding
from .grad_slots import GradSlotRing, GradSlotsPerUnit, GradStagingRing  # noqa: F401
from .optimizer import cpu_adam as _cpu_adam
from .pinned import pinned_empty
from .staging import (  # noqa: F401
    BF16Loader,
    H2DStager,
    LayerBufferPool,
    PendingCast,
    _backlog,
    _new_event,
    overlap_ranges,
    split_into_pieces,
)
from .update_executor import EARLY_UPDATE_PRIORITY, PriorityUpdateExecutor, _UpdateReady  # noqa: F401


def _no_slot() -> None:
    """Offload gate with one slot per unit: nothing to wait for."""
    return None


# The runtime's (h2d, cast, d2h) streams per device index, shared by every
# runtime of the process (see ``runtime_streams``).
_RUNTIME_STREAMS: Dict[int, Tuple[Any, Any, Any]] = {}
_RUNTIME_STREAMS_LOCK = threading.Lock()


def runtime_streams(device: torch.device) -> Tuple[Any, Any, Any]:
    """The ``(h2d, cast, d2h)`` streams of ``device``, made once per process.

    The HIP runtime gives a stream its hardware queue when the stream is
    first used: a new queue while fewer than GPU_MAX_HW_QUEUES exist, then
    the existing ones again.  An event recorded on a stream behind a copy in
    flight holds a packet in that stream's queue until the copy ends, and
    while it is held, kernels of some other queues run slower.  Measured on
    MI355X, the default stream's queue created first: with 8 queues the
    staging cast on the default stream ran at 0.65-0.68 of HBM peak beside
    such a copy from the fifth queue and at 0.75-0.76 beside one from any
    other; with 16 queues it was slow beside the fifth, ninth and
    thirteenth; with 4, beside none.  Copies without an event behind them,
    and SDMA copies issued outside HIP streams, did not slow it.  So the
    default stream and the three streams here are first used together, in
    that order, when they are made: in a process that has used no other
    stream they take the first four queues.  Every later runtime of the
    process reuses them: a second runtime whose streams were new came after
    the first's queues, and its casts ran at 0.64 of peak against 0.74
    when it reused the first's streams (the 2-unit pool schedule after the
    default one, Llama-3-8B).  Sharing the streams between runtimes only
    adds order between their copies.  They come from torch's stream pool
    (32 per device and priority, handed out in turn), so a process that asks
    torch for more streams can be handed one of them for other work, which
    likewise only adds order."""
    dev = torch.device(device)
    key = dev.index if dev.index is not None else torch.cuda.current_device()
    with _RUNTIME_STREAMS_LOCK:
        got = _RUNTIME_STREAMS.get(key)
        if got is None:
            dev = torch.device("cuda", key)
            h2d, cast, d2h = (torch.cuda.Stream(device=dev) for _ in range(3))
            with torch.cuda.device(dev):
                for s in (torch.cuda.current_stream(dev), h2d, d2h, cast):
                    torch.cuda.Event().record(s)   # the stream's first use: its queue
            got = (h2d, cast, d2h)
            _RUNTIME_STREAMS[key] = got
        return got


class StreamingRuntime:
    """Objects shared by all units of one model: streams, pool, stager, grad
    ring, worker threads and the optional event trace."""

    def __init__(self, device: torch.device, dtype: torch.dtype, max_param_size: int, pool_size: int,
                 stage_chunk_elems: int, stage_depth: int, grad_ring_depth: int, wait_timeout: Optional[float],
                 d2h_workgroups: int = 16, d2h_engine: str = "sdma", h2d_format: str = "fp32"):
        if wait_timeout is not None and not wait_timeout > 0:
            raise ValueError("wait_timeout must be a positive number of seconds or None")
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
            # SDMA engine routing coincided with wrong step-1 gradients at
            # full size, cause not found: the runtime does not run with it.
            kernels.require_routing_off()
        # Host AdamW team size (0: leave the library's setting alone); see
        # set_adam_threads.
        self.adam_threads = 0
        # Unit copies the forward and backward may keep queued on the H2D
        # stream before they hold the host (0: no limit); see ``hold_h2d``.
        self.h2d_issue_limit = 0
        self._adam_threads_set = 0
        # Workgroups of the kernels that write into pinned host memory (grad
        # rows and checkpoint offload): 16 move 55-56 GB/s alone and 48-49
        # GB/s in the training step (8: 52-56 and 47), with no measurable
        # cost to the casts and GEMMs beside them; many more slow HBM-bound
        # kernels beside them (the staging cast: 10x beside 64).
        self.d2h_workgroups = d2h_workgroups
        self.h2d_stream, self.cast_stream, self.d2h_stream = runtime_streams(device)
        self.pool = LayerBufferPool(max_param_size, dtype, device, pool_size)
        if h2d_format == "bf16":
            self.stager = BF16Loader(self.h2d_stream)
        else:
            # whole-unit slots of units staged after their update: at most a
            # quarter of the device memory
            cap = torch.cuda.get_device_properties(device).total_memory // 4
            self.stager = H2DStager(device, stage_chunk_elems, stage_depth, self.h2d_stream, self.cast_stream,
                                    slot_cap_bytes=cap)
        # bf16 copies on the H2D stream: the loads of bf16 H2D, or the
        # backward's reloads of units with a bf16 reload copy (fp32 H2D); its
        # copies are timed in the stager's list
        self.bf16_loader = (self.stager if h2d_format == "bf16"
                            else BF16Loader(self.h2d_stream, timing_source=self.stager))
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
        # fp32 H2D: units are copied whole into a device fp32 slot and cast
        # where they are next used, on that stream between its kernels,
        # instead of on the cast stream as soon as their copy lands.
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
        # pack and the update against the oracle, and for every unit but the
        # row-sparse embedding {("grad_sums", unit): [int64 sum of each
        # gradient's 16-bit words]}.  ``capture_units`` (a set)
        # limits it to those units (None: every unit), so that full-size
        # models capture a few units instead of copying every one.
        self.capture: Optional[dict] = None
        self.capture_units: Optional[set] = None
        # Test hook: when a dict, device copies of the checkpoint tensors each
        # recompute is given, {(decoder index, tensor index): tensor}.
        self.capture_served: Optional[dict] = None
        self._held: List[Any] = []
        # Optional measurement: when a dict (``enable_link_timing``), timing
        # events of the units' compute on the compute stream and of the host
        # link work besides the parameter and gradient copies (checkpoint
        # packs and prefetches, embedding row gathers).
        self.link_timing: Optional[Dict[str, Any]] = None

    def enable_link_timing(self, on: bool = True) -> None:
        """Start (or stop) recording the intervals ``link_timing`` holds:
        "compute" [(start, end)] events around each unit's forward and
        backward on the compute stream, and (start, end, bytes) events of
        "act_d2h" / "act_h2d" (checkpoint packs and prefetches) and
        "rows_h2d" / "rows_d2h" (embedding row gathers)."""
        self.link_timing = ({"compute": [], "act_d2h": [], "act_h2d": [], "rows_h2d": [], "rows_d2h": []}
                            if on else None)

    def compute_mark(self, start: bool) -> None:
        """With link timing on, a timing event on the current stream that
        opens (``start``) or closes a unit's compute interval."""
        lt = self.link_timing
        if lt is None:
            return
        ev = torch.cuda.Event(enable_timing=True)
        ev.record(torch.cuda.current_stream())
        if start:
            lt["_open"] = ev
        else:
            first = lt.pop("_open", None)
            if first is not None:
                lt["compute"].append((first, ev))

    def hold_forever(self, objs) -> None:
        """Keep ``objs`` referenced until the process ends: the host slot and
        the device tensors of copies that never completed, which an engine
        may still write into or read from."""
        self._held.append(objs)

    def capturing(self, unit: int) -> bool:
        """True if the test hook ``capture`` records ``unit``."""
        return self.capture is not None and (self.capture_units is None or unit in self.capture_units)

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
        few = self.h2d_backlog() >= 2
        n = max(1, (self.adam_threads + 1) // 2) if few else self.adam_threads
        if n != self._adam_threads_set:
            _cpu_adam.set_num_threads(n)
            self._adam_threads_set = n

    def h2d_backlog(self) -> int:
        """Host-to-device unit copies issued and not yet complete."""
        n = self.stager.backlog()
        if self.bf16_loader is not self.stager:
            n += self.bf16_loader.backlog()
        return n

    def hold_h2d(self, what: str) -> None:
        """Before the forward or the backward issues a unit copy: while
        ``h2d_issue_limit`` or more unit copies are queued, wait for the
        oldest to complete (bounded by the wait limit).  A queued HIP copy
        holds an SDMA engine until it has run, and the HIP runtime puts each
        new copy on the first engine not held: with many copies queued, the
        later ones land on engines that copy slower."""
        limit = self.h2d_issue_limit
        if not limit:
            return
        while self.h2d_backlog() >= limit:
            oldest = None
            for q in (self.stager._copies, self.bf16_loader._copies):
                try:
                    oldest = q[0]   # other threads may trim the queue meanwhile
                    break
                except IndexError:
                    continue
            if oldest is None:
                return
            kernels.wait_event(oldest, self.wait_timeout, what)

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
        """Finish the queued offloads and updates and stop both worker
        threads (each join bounded by ``wait_timeout``)."""
        try:
            if self.offload_executor is not None:
                self.offload_executor.shutdown(wait=True, timeout=self.wait_timeout)
        finally:
            self.update_executor.shutdown(wait=True, timeout=self.wait_timeout)

    def release_slots(self, states) -> None:
        """Give back the whole-unit slots of stagings not yet cast (their units
        are then staged from the master if used again) and free the pool's
        buffers once the copy and cast streams have drained and each slot's
        last cast (on the forward's stream, with casts at use) has
        completed."""
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
        slots.release(self.wait_timeout)


class LayerRuntimeState(RowSparseEmbedding, nn.Module):
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
        # fp32 H2D, units reloaded for their backward: a pinned bf16 copy of
        # the master that the update keeps current (``enable_bf16_reload``).
        self._reload_bf16: Optional[torch.Tensor] = None
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
        """Recompute the bf16 host copy from the fp32 master (bf16 H2D, or the
        backward's bf16 reload copy) and drop a staging made for the next
        forward.  Updates keep both current; call this after writing the
        master directly."""
        self._drop_prefetched()
        host = self._bf16_host()
        if host is not None and self.total_size:
            _cpu_adam.cast_f32_bf16(self._cpu_params_flat, host)

    def _bf16_host(self) -> Optional[torch.Tensor]:
        """The pinned bf16 copy of the master that updates rewrite, if any."""
        return self._cpu_params_bf16 if self._cpu_params_bf16 is not None else self._reload_bf16

    def enable_bf16_reload(self) -> bool:
        """fp32 H2D: keep a pinned bf16 copy of this unit's master, written by
        each update in the same pass, and reload the unit for its backward
        from it: 2 bytes per parameter over the host link instead of 4, and
        no cast.  Same bits: the master does not change between a unit's
        forward and its backward, and the copy is the RNE cast of it.  Returns
        False (the unit keeps reloading fp32) when the host cannot pin it."""
        if (self._reload_bf16 is not None or self._cpu_params_bf16 is not None or self.row_sparse
                or not self.backward_reads_params or self.buffer_pool.dtype != torch.bfloat16
                or self.runtime.h2d_format != "fp32" or not self.total_size):
            return self._reload_bf16 is not None
        try:
            copy = pinned_empty(self.total_size, torch.bfloat16)
        except _native.NativeError as e:
            if e.status != _native.HIP_ERROR_OUT_OF_MEMORY:
                raise
            return False
        self.wait_for_update()
        with self.update_lock:
            _cpu_adam.cast_f32_bf16(self._cpu_params_flat, copy)
            self._reload_bf16 = copy
        return True

    def _drop_prefetched(self) -> None:
        """Forget a staging made for the next forward (its master changed): a
        copy not cast yet gives its slot back; a cast already issued becomes
        the unit's last writer, which the next staging into it waits for."""
        with self._prefetch_lock:
            old, self._prefetched = self._prefetched, None
        if old is None:
            return
        unit, done = old
        if isinstance(done, PendingCast):
            self.runtime.stager.drop_pending(done)
        elif done is not None:
            unit["ready"] = done

    def release_device_unit(self) -> None:
        """Give back this unit's device buffer if it is still loaded (after a
        forward without a backward, units with a buffer of their own, the
        last decoder and the output unit stay loaded) and point its
        parameters at their fp32 master views again; drop a pending cast and
        a staging made for the next forward.  Call before writing the
        master directly: while the unit is loaded, ``param.data`` is its bf16
        device view and a write there would not reach the master."""
        unit = self._current_gpu_cache
        if unit is not None:
            self._drop_pending_cast()
            ev = _new_event()
            ev.record(torch.cuda.current_stream())
            unit["ready"] = ev
            self._bind_host_views()
            self._current_gpu_cache = None
            self._bwd_armed = False
            self._release_unit(unit)
        self._drop_prefetched()

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
        if not skip:
            self.runtime.hold_h2d(f"unit {self.layer_idx}: queued copies before its load")
        if self._cpu_params_bf16 is not None:
            unit = self._acquire_unit()
            self._h2d_done = unit["ready"] if skip else stager.load(self._cpu_params_bf16, unit["param"], unit["ready"])
            self._bind_unit(unit, is_backward)
            return
        if is_backward and not skip and self._reload_bf16 is not None:
            # the backward's reload: the bf16 copy the last update wrote
            unit = self._acquire_unit()
            self._drop_pending_cast()
            self._h2d_done = self.runtime.bf16_loader.load(self._reload_bf16, unit["param"], unit["ready"])
            self._bind_unit(unit, is_backward)
            return
        if not skip and self.runtime.cast_at_use:
            # The whole unit is copied into a device fp32 slot now, before the
            # pool wait, and cast where it is used (``wait_for_h2d``, on the
            # forward's or the backward's stream right before the unit's
            # kernels), so the cast does not share the HBM with the GEMMs of
            # the unit computing meanwhile.
            pc = stager.copy_for_later(self._cpu_params_flat, None)
            if pc is not None:
                try:
                    unit = self._acquire_unit()
                except BaseException:
                    stager.drop_pending(pc)
                    raise
                pc.wait_event = unit["ready"]   # the unit's previous reader
                self._drop_pending_cast()
                self._pending_cast, self._h2d_done = pc, None
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
        try:
            return self.buffer_pool.acquire(timeout=self.runtime.wait_timeout)
        except TimeoutError as e:
            raise TimeoutError(f"Layer {self.layer_idx}: {e}") from None

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
        # Taken on the cast stream, which writes it, so that neither pending
        # work of another stream on the block nor its release after the cast
        # is left unordered.
        with torch.cuda.stream(self.runtime.cast_stream):
            return torch.empty(self.total_size, dtype=self.buffer_pool.dtype, device=self.runtime.device)

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
        if self.runtime.capturing(self.layer_idx):
            self.runtime.capture[("device_grads", self.layer_idx)] = [
                None if p.grad is None else p.grad.detach().clone() for p in self._params]
        if self.runtime.capture is not None:
            # every unit, also outside ``capture_units``: the sum of each
            # gradient's 16-bit words (exact, a few bytes per parameter)
            self.runtime.capture[("grad_sums", self.layer_idx)] = [
                None if p.grad is None else p.grad.detach().view(torch.int16).sum(dtype=torch.int64)
                for p in self._params]
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
        issued: List[Any] = []   # SDMA copies started so far (not stream-ordered)
        try:
            host = rt.grad_ring.slots[slot]
            pairs = [(g, host[off:off + g.numel()]) for g, off in grads]
            if rt.d2h_engine == "sdma":
                # The gradients must be complete before an SDMA engine reads
                # them (the copy is not stream-ordered): wait here, on this
                # worker thread, then hand the copy to the engine.
                kernels.wait_event(grad_ready, rt.wait_timeout, f"unit {self.layer_idx}: gradients")
                rt.mark("grad_ready", self.layer_idx)
                plan = self._piece_plan()
                if plan is None:
                    issued.append(kernels.dma_copy_d2h(pairs, timeout=rt.wait_timeout))
                else:
                    # one copy per piece, in update order: the update starts
                    # once the first has landed
                    spans = [(off, g.numel()) for g, off in grads]
                    for a, b in plan[0]:
                        sub = [(grads[i][0][lo:hi], host[grads[i][1] + lo:grads[i][1] + hi])
                               for i, lo, hi in overlap_ranges(spans, a, b)]
                        issued.append(kernels.dma_copy_d2h(sub, timeout=rt.wait_timeout) if sub else None)
                rt.mark("dma_issued", self.layer_idx)
                done = None
                dma_ready = [None if h is None else kernels.DmaReady(h, timeout=rt.wait_timeout) for h in issued]
                handle = issued
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
            nbytes = 2 * sum(g.numel() for g, _ in grads)
            # With SDMA the gradient tensors stay referenced until the copy is
            # waited for; the caching allocator cannot hand them out before then.
            keep = grads if handle is not None else None
            if handle is None:
                ready = done
            else:
                ready = next((d for d in dma_ready if d is not None), None)
            self._update_future = rt.update_executor.submit(
                rt.update_priority(self.layer_idx), self._do_update, slot, done, missing,
                None if handle is None else dma_ready, keep, nbytes, ready=self._update_ready(ready))
        except BaseException:
            self._abandon_copies(issued, grads, slot)
            raise

    def _abandon_copies(self, issued, grads, slot) -> None:
        """After a failed offload: the SDMA copies already started must land
        before the host slot is handed back and the gradients are freed.
        Copies that do not complete within the wait limit keep both for the
        life of the process (an engine may still write into the slot)."""
        rt = self.runtime
        try:
            for h in issued:
                if h is not None:
                    kernels.DmaReady(h, timeout=rt.wait_timeout).release()
            if rt.d2h_engine != "sdma":
                # stream-ordered copies that may have been enqueued
                drained = _new_event()
                drained.record(rt.d2h_stream)
                kernels.wait_event(drained, rt.wait_timeout, f"unit {self.layer_idx}: gradient copies")
        except TimeoutError:
            rt.hold_forever((grads, issued, slot))
        else:
            rt.grad_ring.release(slot)
        finally:
            self.update_finished.set()

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
        host = self._bf16_host()
        if host is None:
            return None
        return self._grad_views(host)

    def _grad_views(self, host: torch.Tensor) -> Dict[nn.Parameter, torch.Tensor]:
        views = {}
        for (name, (off, shape, size)), p in self._named():
            views[p] = host[off:off + size].view(shape)
        return views

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
                kernels.wait_event(d2h_done, rt.wait_timeout, f"unit {self.layer_idx}: gradient copy")
            plan = self._piece_plan() if self.layer_optimizer is not None else None
            if plan is None or len(chunks) not in (0, len(plan[0])):
                wait_chunks(len(chunks))
            for off, size in missing:
                # a parameter that received no gradient: zeros, as the zeroed
                # grad buffer of the reference gives it (layer_state.py:297);
                # no copy writes these ranges
                rt.grad_ring.slots[slot][off:off + size].zero_()
            master_before = self._cpu_params_flat.clone() if rt.capturing(self.layer_idx) else None
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
                # and the gradients are freed
                try:
                    wait_chunks(len(chunks))
                except kernels.DmaCopiesOutstanding:
                    rt.hold_forever((keep, chunks, slot))
                    raise
                del keep
                if rt.d2h_timing is not None and state["t0"] is not None:
                    rt.d2h_timing.append(("interval_ns", state["t0"], state["t1"], nbytes))
                elif rt.d2h_timing is not None and any(ch is not None for ch in chunks):
                    # SDMA copies without engine timestamps (a profiler that
                    # traces async copies takes them over)
                    rt.d2h_timing.append(("untimed", nbytes))
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
        for what, f in (("gradient offload", self._d2h_future), ("parameter update", self._update_future)):
            if f is None:
                continue
            try:
                f.result(timeout=t)
            except futures.TimeoutError:
                raise TimeoutError(f"Layer {self.layer_idx} {what} not finished after {t:g} s") from None
        if not self.update_finished.wait(timeout=t):
            raise TimeoutError(f"Layer {self.layer_idx} parameter update timed out")

    def forward(self, *args, **kwargs):
        raise NotImplementedError("LayerRuntimeState manages state; call .layer(...) for compute")
