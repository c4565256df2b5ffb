"""The runtime's device-side ordering, checked on the CPU with the
happens-before model of ``hb_model``: the real staging, pool, checkpoint and
gradient-offload code runs against stand-in streams, events, device memory
(with a model of torch's caching allocator) and copy/cast entry points, and
every pair of conflicting accesses must be ordered by device events or by a
host wait on them, never by host timing alone.

Each protocol is checked as the runtime runs it and with one planted mistake
(the ordering it depends on taken away), which the model must report:

* whole-unit fp32 slots taken while the backward frees memory: allocated on
  the stream that copies into them (a slot taken on the compute stream, the
  earlier code, reuses a block the backward's queued kernels still use);
* the 2-unit pool and the chunk ring of the stager: each cast waits for its
  unit's last reader and each copy for its ring slot's last cast;
* a pool unit copied whole and cast where it is used (forward and backward
  reloads, ``to_device_async`` / ``wait_for_h2d``);
* checkpoint packs and the two-set prefetch ring of ``SlidingCheckpoint``:
  the pack source kept from reuse by ``record_stream``, a ring set refilled
  only after the recompute that read it, each prefetch ordered after its
  decoder's last pack (an event), and with SDMA packs the copy started after
  its source's producer, the source held and the slot read only after the
  copy was seen complete;
* gradient offload on SDMA engines (``_d2h_task`` / ``_do_update``): the copy
  reads the gradients after their event, the host AdamW reads the slot after
  the copy, and the slot and the gradients' memory are reused only after it;
* no pinned allocation inside the forward while a host copy is in flight."""

import threading
from types import SimpleNamespace

import pytest
import torch

import hb_model
from hb_model import Device, FakeEvent

N = 4096


@pytest.fixture
def dev(monkeypatch):
    from test1_amd import layer_state, sliding_checkpoint, staging

    d = Device()
    hb_model.install(monkeypatch, d, staging, layer_state, sliding_checkpoint)
    return d


def _stager(dev, chunk=N, depth=3, slot_cap=1 << 30):
    from test1_amd.staging import H2DStager

    h2d, cast = hb_model.FakeStream(dev, "h2d"), hb_model.FakeStream(dev, "cast")
    return H2DStager("cuda:0", chunk, depth, h2d, cast, slot_cap_bytes=slot_cap)


# ---------------------------------------------------------------------------
# Whole-unit slots taken by the update thread during the backward
# ---------------------------------------------------------------------------

def _stage_after_update_while_backward_frees(dev, stager):
    comp = dev.default
    master = torch.randn(N)
    # the backward: an activation written and read by kernels still queued on
    # the compute stream, its memory freed by the autograd thread meanwhile
    with dev.as_host("autograd"):
        act = dev.alloc((N,), torch.float32)
        dev.op(comp, writes=[act], what="backward kernel writing an activation")
        dev.op(comp, reads=[act], what="backward kernel reading it")
        dev.free(act)
    # the update thread stages the updated unit for the next forward
    with dev.as_host("update"):
        pc = stager.copy_for_later(master, None)
    assert pc is not None
    # the next forward casts it where it is used
    with dev.as_host("autograd"):
        unit = dev.alloc((N,), torch.bfloat16)
        stager.cast_pending(pc, unit, comp)
        dev.op(comp, reads=[unit], what="forward reading the unit")


def test_whole_unit_slot_allocated_on_the_copy_stream(dev):
    _stage_after_update_while_backward_frees(dev, _stager(dev))
    assert dev.races == []


def test_whole_unit_slot_allocated_on_the_compute_stream_races(dev):
    """The ordering before the fix: the slot came from the update thread's
    current stream, the compute stream, and took the activation's block."""
    st = _stager(dev)
    st.slots.alloc_stream = None
    _stage_after_update_while_backward_frees(dev, st)
    assert any("copy on h2d" in r and "backward kernel" in r for r in dev.races), dev.races


# ---------------------------------------------------------------------------
# The 2-unit pool and the chunk ring: begin/finish with the unit's fence
# ---------------------------------------------------------------------------

def _stream_units(dev, stager, L=6, fence=True):
    from test1_amd.staging import LayerBufferPool

    comp = dev.default
    pool = LayerBufferPool(N, torch.bfloat16, "cuda:0", 2)
    masters = [torch.randn(N) for _ in range(L)]
    for i in range(L):
        unit = pool.acquire(timeout=1)
        done = stager.load(masters[i], unit["param"], unit["ready"] if fence else None)
        comp.wait_event(done)
        dev.op(comp, reads=[unit["param"]], what=f"layer {i} forward")
        ev = FakeEvent()
        ev.record(comp)
        unit["ready"] = ev
        pool.release(unit)


@pytest.mark.parametrize("chunk,depth", [(N, 3), (N // 4, 2), (N // 3, 3)])
def test_pool_units_through_the_chunk_ring(dev, chunk, depth):
    _stream_units(dev, _stager(dev, chunk, depth))
    assert dev.races == []


def test_cast_without_the_units_fence_races(dev):
    """The reference's ordering (layer_state.py:292-315): the next H2D into a
    unit released on the host, without waiting for the compute stream."""
    _stream_units(dev, _stager(dev), fence=False)
    assert any("cast on cast" in r and "forward" in r for r in dev.races), dev.races


def test_ring_copy_without_its_slot_fence_races(dev):
    st = _stager(dev, N // 4, 2)
    dev.skip_waits["h2d"] = True      # the copies no longer wait for the slot's last cast
    _stream_units(dev, st)
    assert any("copy on h2d" in r and "cast on cast" in r for r in dev.races), dev.races


# ---------------------------------------------------------------------------
# A pool unit copied whole and cast where it is used (LayerRuntimeState)
# ---------------------------------------------------------------------------

def _unit_state(dev, idx, runtime, master):
    from test1_amd import layer_state

    st = object.__new__(layer_state.LayerRuntimeState)
    st.__dict__.update(
        layer_idx=idx, runtime=runtime, buffer_pool=runtime.pool, row_sparse=False, _own_unit=None,
        _current_gpu_cache=None, _prefetched=None, _prefetch_lock=threading.Lock(), _pending_cast=None,
        _h2d_done=None, _cpu_params_bf16=None, _cpu_params_flat=master, backward_reads_params=True,
        _param_maps={}, _params=[], _bwd_compute_done=False, _grads_offloaded=False, _reload_bf16=None)
    st.wait_for_update = lambda timeout=None: None
    return st


def _runtime(dev, stager, pool_size=2, h2d_issue_limit=0):
    from types import MethodType

    from test1_amd.layer_state import StreamingRuntime
    from test1_amd.staging import BF16Loader, LayerBufferPool

    rt = SimpleNamespace(stager=stager, pool=LayerBufferPool(N, torch.bfloat16, "cuda:0", pool_size),
                         bf16_loader=BF16Loader(stager.h2d_stream, timing_source=stager),
                         cast_at_use=True, wait_timeout=1.0, log=lambda *a: None, mark=lambda *a: None,
                         h2d_issue_limit=h2d_issue_limit)
    rt.h2d_backlog = MethodType(StreamingRuntime.h2d_backlog, rt)
    rt.hold_h2d = MethodType(StreamingRuntime.hold_h2d, rt)
    return rt


def _pool_step(dev, rt, states):
    """One step of the reference's schedule through ``to_device_async`` /
    ``wait_for_h2d``: forward loads one ahead, backward reloads the unit
    below before each unit's backward, units released after their use."""
    L = len(states)
    comp = dev.default
    # forward: the next unit's load issued before this unit's forward
    states[0].to_device_async()
    for i, st in enumerate(states):
        if i + 1 < L:
            states[i + 1].to_device_async()
        assert st._pending_cast is not None          # copied, not cast yet
        st.wait_for_h2d()
        dev.op(comp, reads=[st._current_gpu_cache["param"]], what=f"unit {i} forward")
        if i < L - 1:
            st.to_offload_async(is_backward=False)
    # backward: reload the unit below before this unit's backward
    for i in range(L - 1, -1, -1):
        st = states[i]
        if i - 1 >= 0:
            states[i - 1].to_device_async(is_backward=True)
        st.wait_for_h2d()
        dev.op(comp, reads=[st._current_gpu_cache["param"]], what=f"unit {i} backward")
        st._bwd_compute_done = st._grads_offloaded = True
        st._maybe_release_after_backward()


@pytest.mark.parametrize("issue_limit", [0, 1, 2])
def test_pool_loads_cast_at_use_forward_and_backward(dev, issue_limit):
    """The pool step, also with the host held while ``issue_limit`` unit
    copies are queued (the hold only waits for issued copies)."""
    rt = _runtime(dev, _stager(dev), h2d_issue_limit=issue_limit)
    _pool_step(dev, rt, [_unit_state(dev, i, rt, torch.randn(N)) for i in range(5)])
    assert dev.races == []
    assert rt.pool.available() == 2


def test_backward_reloads_from_the_bf16_copy(dev):
    """Units with a bf16 reload copy: the forward's fp32 copy and cast at
    use, the backward's bf16 copy straight into the pool unit after the
    unit's last reader."""
    rt = _runtime(dev, _stager(dev))
    states = [_unit_state(dev, i, rt, torch.randn(N)) for i in range(5)]
    for st in states:
        st._reload_bf16 = torch.zeros(N, dtype=torch.bfloat16)
    _pool_step(dev, rt, states)
    assert dev.races == []
    assert rt.pool.available() == 2
    assert any("copy on h2d" in a[5] and a[4] for a in dev.accesses)


def test_backward_bf16_reload_without_the_units_fence_races(dev, monkeypatch):
    from test1_amd.staging import BF16Loader

    rt = _runtime(dev, _stager(dev))
    real = BF16Loader.load
    monkeypatch.setattr(BF16Loader, "load", lambda self, h, d, w: real(self, h, d, None))
    states = [_unit_state(dev, i, rt, torch.randn(N)) for i in range(5)]
    for st in states:
        st._reload_bf16 = torch.zeros(N, dtype=torch.bfloat16)
    _pool_step(dev, rt, states)
    assert any("copy on h2d" in r and "forward" in r for r in dev.races), dev.races


# ---------------------------------------------------------------------------
# Checkpoint packs and the two-set prefetch ring
# ---------------------------------------------------------------------------

def _checkpoint_round_trip(dev, L=6, shape=(2, 8, 64), one_set=False, drop_record_stream=False,
                           before_pin=None, pin_check=None, monkeypatch=None, pack_engine="kernel",
                           free_sources_early=None, drain_before_pin=False):
    """L decoders' checkpoints packed in the forward (kernel on the D2H stream
    or SDMA copies issued by the ring's worker) and prefetched back on the
    H2D stream in the backward, the host slots' ranges tracked as well.  The
    autograd graph keeps only the packed copy: a source is freed right after
    its pack (the kernel path; its ``record_stream`` fences the reuse) or
    once the ring has released it (the SDMA path)."""
    from test1_amd import sliding_checkpoint as sc_mod
    from test1_amd.sliding_checkpoint import ActivationRing, SlidingCheckpoint

    dev.track_host = True
    if free_sources_early is None:
        free_sources_early = pack_engine == "kernel"
    if monkeypatch is not None:
        def pinned(shape_, dtype):
            if pin_check is not None:
                pin_check()
            return torch.empty(shape_, dtype=dtype)
        monkeypatch.setattr(sc_mod, "pinned_empty", pinned)
        if one_set:
            real = ActivationRing.buffers_like

            def same_set(self, host):
                self.next = 0
                return real(self, host)
            monkeypatch.setattr(ActivationRing, "buffers_like", same_set)
        if drop_record_stream:
            monkeypatch.setattr(hb_model.DevTensor, "record_stream", lambda self, s: None)
    comp = dev.default
    d2h, h2d = hb_model.FakeStream(dev, "d2h"), hb_model.FakeStream(dev, "h2d")
    ring = ActivationRing("cuda:0")
    if drain_before_pin:
        def before_pin():
            dev.synchronize()
            ring.drain_packs()
    slots = [[None] for _ in range(L)]
    scs, packed, held = [], [], []
    x = dev.alloc(shape, torch.bfloat16)
    dev.op(comp, writes=[x], what="embedding writing the first layer's input")
    try:
        for i in range(L):
            sc = SlidingCheckpoint(layer_idx=i + 1, layer_tensors=slots, is_last_layer=(i == L - 1), no_mask=True,
                                   device="cuda:0", stream=d2h, prefetch_stream=h2d, prefetch_ring=ring,
                                   before_pin=before_pin, pack_engine=pack_engine)
            packed.append(sc.pack_hook(x))
            scs.append(sc)
            y = dev.alloc(shape, torch.bfloat16)
            dev.op(comp, reads=[x], writes=[y], what=f"layer {i} forward")
            if i < L - 1:
                if free_sources_early:
                    dev.free(x)   # the autograd graph keeps only the packed copy
                else:
                    held.append(x)
            x = y
        for i in range(L - 1, -1, -1):
            t = scs[i].unpack_hook(packed[i])
            dev.op(comp, reads=[t], what=f"layer {i} recompute")
            tmp = dev.alloc(shape, torch.bfloat16)      # the recompute's own activations
            dev.op(comp, writes=[tmp], what=f"layer {i} backward")
            dev.free(tmp)
    finally:
        ring.close()
    return slots


@pytest.mark.parametrize("free_sources_early", [True, False])
def test_checkpoint_round_trip_is_ordered(dev, monkeypatch, free_sources_early):
    _checkpoint_round_trip(dev, monkeypatch=monkeypatch, free_sources_early=free_sources_early)
    assert dev.races == []


def test_checkpoint_prefetch_without_the_pack_event_races(dev, monkeypatch):
    """The prefetch on the H2D stream reads a host slot that the pack kernel
    on the D2H stream wrote: without the event recorded after the decoder's
    last pack the two copies are unordered.  (They were ordered only while
    both ran on one stream, or when the source's memory happened to be
    reused first: the caching allocator then waits for the pack; here the
    sources stay allocated.)"""
    from test1_amd.sliding_checkpoint import ActivationRing

    class _Forgetful(dict):
        def __setitem__(self, k, v):
            pass

    real_init = ActivationRing.__init__

    def init(self, *a, **kw):
        real_init(self, *a, **kw)
        self.packed_events = _Forgetful()
    monkeypatch.setattr(ActivationRing, "__init__", init)
    _checkpoint_round_trip(dev, monkeypatch=monkeypatch, free_sources_early=False)
    assert any("copy on h2d" in r and "pack on d2h" in r for r in dev.races), dev.races


def test_checkpoint_round_trip_on_sdma_is_ordered(dev, monkeypatch):
    """Packs by SDMA copies: each starts after its source's producer (a host
    wait on the compute stream's event), the prefetch reads the slot after
    the copy was seen complete, and the source is freed only then."""
    _checkpoint_round_trip(dev, monkeypatch=monkeypatch, pack_engine="sdma")
    assert dev.races == []


def test_checkpoint_sdma_prefetch_without_settling_races(dev, monkeypatch):
    from test1_amd.sliding_checkpoint import ActivationRing

    monkeypatch.setattr(ActivationRing, "settle_packs", lambda self, key, layer, timing=None: None)
    _checkpoint_round_trip(dev, monkeypatch=monkeypatch, pack_engine="sdma")
    assert any("copy on h2d" in r and "SDMA copy" in r for r in dev.races), dev.races


def test_checkpoint_sdma_source_freed_before_its_copy_races(dev, monkeypatch):
    """The autograd graph drops a checkpoint's source after the pack; the
    ring must keep it until its SDMA copy has been seen complete."""
    _checkpoint_round_trip(dev, monkeypatch=monkeypatch, pack_engine="sdma", free_sources_early=True)
    assert any("forward" in r and "SDMA copy" in r for r in dev.races), dev.races


def test_prefetch_ring_of_one_set_races(dev, monkeypatch):
    """A one-set ring: layer j-1's prefetch would overwrite layer j's
    checkpoint before layer j's recompute has read it."""
    _checkpoint_round_trip(dev, one_set=True, monkeypatch=monkeypatch)
    assert any("copy on h2d" in r and "recompute" in r for r in dev.races), dev.races


def test_pack_source_without_record_stream_races(dev, monkeypatch):
    """The reference's pack (sliding_checkpoint.py:69-73) does not fence the
    source: its memory can be reused on the compute stream while the
    offload stream still reads it."""
    _checkpoint_round_trip(dev, drop_record_stream=True, monkeypatch=monkeypatch)
    assert any("pack on d2h" in r for r in dev.races), dev.races


@pytest.mark.parametrize("pack_engine", ["kernel", "sdma"])
def test_checkpoint_slots_pinned_only_with_no_host_copy_in_flight(dev, monkeypatch, pack_engine):
    """Slots pinned inside the forward (first step, new batch shape) are
    pinned after ``before_pin`` (the model drains its copies there: the
    device and the ring's SDMA packs), never while a copy into or out of
    host memory is in flight."""
    def check():
        assert dev.outstanding_host_copies() == [], "pinned while host copies were in flight"

    _checkpoint_round_trip(dev, pin_check=check, monkeypatch=monkeypatch, pack_engine=pack_engine,
                           drain_before_pin=True)
    assert dev.races == []


def test_checkpoint_slots_pinned_without_draining_are_caught(dev, monkeypatch):
    def check():
        assert dev.outstanding_host_copies() == [], "pinned while host copies were in flight"

    with pytest.raises(AssertionError, match="pinned while host copies"):
        _checkpoint_round_trip(dev, before_pin=None, pin_check=check, monkeypatch=monkeypatch)


# ---------------------------------------------------------------------------
# Gradient offload on SDMA engines: _d2h_task and _do_update
# ---------------------------------------------------------------------------

class _OneSlotRing:
    """One pinned gradient slot; a release orders the next acquire after
    everything the releasing thread had seen (the ring's lock)."""

    def __init__(self, dev, n):
        self.dev = dev
        self.slots = {0: torch.zeros(n, dtype=torch.bfloat16)}
        self.free = True
        self.clock = hb_model.VC()

    def acquire(self, timeout=None, unit=None):
        assert self.free, "slot taken twice"
        self.free = False
        self.dev.host().join(self.clock)
        return 0

    def release(self, idx):
        self.clock = self.dev.host().copy()
        self.free = True


class _HostOptimizer:
    """The host AdamW's accesses: it reads the slot's gradient views."""

    def __init__(self, dev):
        self.dev = dev

    def step_with_grad_views(self, idx, views, **kw):
        for v in views.values():
            self.dev.host_read(v, f"host AdamW of unit {idx}")


def _grad_offload(dev, units=3, skip_dma_waits=False):
    """Three units' gradients through ``_d2h_task`` (offload thread: wait for
    the gradients' event, SDMA copies into the one host slot) and
    ``_do_update`` (update thread: wait for the copies, the host AdamW reads
    the slot, the slot goes back), the gradients' memory freed after each
    update and reused for the next unit's gradients."""
    from test1_amd import layer_state

    comp = dev.default
    ring = _OneSlotRing(dev, N)
    queued = []
    rt = SimpleNamespace(grad_ring=ring, wait_timeout=1.0, d2h_engine="sdma", mark=lambda *a: None,
                         piece_elems=0, update_priority=lambda u: u, d2h_timing=None, capture=None, stage_after_update=False,
                         capturing=lambda u: False, set_adam_threads=lambda: None, hold_forever=lambda o: None,
                         update_executor=SimpleNamespace(
                             submit=lambda prio, fn, *a, ready=None: queued.append((fn, a))))
    opt = _HostOptimizer(dev)
    dev.skip_dma_waits = skip_dma_waits
    for unit in range(units):
        with dev.as_host("autograd"):
            g = dev.alloc((N,), torch.bfloat16)
            dev.op(comp, writes=[g], what=f"backward writing unit {unit}'s gradient")
            ev = FakeEvent()
            ev.record(comp)
        st = object.__new__(layer_state.LayerRuntimeState)
        p = torch.nn.Parameter(torch.zeros(N))
        st.__dict__.update(runtime=rt, layer_idx=unit, layer_optimizer=opt, update_finished=threading.Event(),
                           update_lock=threading.Lock(), _param_maps={"w": (0, torch.Size([N]), N)}, _params=[p],
                           _param_views={"w": p.data}, _cpu_params_flat=p.data, _cpu_params_bf16=None,
                           _reload_bf16=None, _plan_key=0, _plan=None, total_size=N)
        st._update_ready = lambda ready: ready
        with dev.as_host("offload"):
            st._d2h_task(None, [(g, 0)], [], ev, None)
        fn, args = queued.pop()
        with dev.as_host("update"):
            fn(*args)
            dev.free(g)        # the last reference to the gradient goes with the update task


def test_gradient_offload_is_ordered(dev):
    _grad_offload(dev)
    assert dev.races == []


def test_gradient_slot_read_before_the_copy_lands_races(dev):
    """An update (and a slot reuse) that does not wait for the SDMA copies:
    the host AdamW reads the slot while an engine may still write it."""
    _grad_offload(dev, skip_dma_waits=True)
    assert any("host AdamW" in r and "SDMA copy" in r for r in dev.races), dev.races
    assert any("backward writing" in r and "SDMA copy" in r for r in dev.races), dev.races


# ---------------------------------------------------------------------------
# SlideFSDP's step preamble: every pinned allocation after a drain
# ---------------------------------------------------------------------------

def _preamble_model(monkeypatch, events, row_sparse=True, ring_pending=False):
    from test1_amd import slide_fsdp

    sf = object.__new__(slide_fsdp.SlideFSDP)
    emb = SimpleNamespace(row_sparse=row_sparse, buffers=0)
    emb.host_buffers_fit = lambda ntok: emb.buffers >= ntok
    emb.has_host_buffers = lambda: emb.buffers > 0

    def alloc_rows(ntok):
        events.append("pin rows")
        emb.buffers = ntok

    emb.alloc_host_buffers = alloc_rows
    sf.__dict__.update(model_config=SimpleNamespace(hidden_size=8), layer_states=[emb], layer_tensors=None,
                       num_decoder_layers=3, dtype=torch.bfloat16, _ring_grow_pending=ring_pending,
                       config=SimpleNamespace(ac_offload_mode="cpu", enable_activation_checkpoint=True))
    sf.__dict__["_drain"] = lambda: events.append("drain")
    sf.__dict__["_grow_grad_ring"] = lambda: events.append("pin ring")

    def pin(shape, dtype):
        events.append("pin slot")
        return torch.empty(shape, dtype=dtype)

    monkeypatch.setattr(slide_fsdp, "pin_or_keep", pin)
    return sf


def _pins_follow_drains(events):
    drained = False
    for e in events:
        if e == "drain":
            drained = True
        elif e.startswith("pin"):
            assert drained, f"{e} without a drain before it: {events}"
        else:
            drained = False       # a step ran copies after the drain


@pytest.mark.parametrize("row_sparse", [True, False])
def test_step_preamble_pins_only_after_draining(monkeypatch, row_sparse):
    events = []
    sf = _preamble_model(monkeypatch, events, row_sparse=row_sparse)
    # an evaluation forward may have left copies in flight before the first training step
    events.append("copies in flight")
    sf._prepare_host_buffers(2, 16)                  # first step: slots and row buffers
    events.append("copies in flight")
    sf._prepare_host_buffers(2, 16)                  # same shape: nothing pinned
    events.append("copies in flight")
    sf._ring_grow_pending = True
    sf._prepare_host_buffers(4, 16)                  # ring growth and a larger batch
    _pins_follow_drains(events)
    pins = [e for e in events if e.startswith("pin")]
    assert pins.count("pin slot") == 2 * sf.num_decoder_layers and pins.count("pin ring") == 1
    assert pins.count("pin rows") == (2 if row_sparse else 0)
    assert events[1] == "drain"                      # drained on the very first step too


# ---------------------------------------------------------------------------
# Slots given back at close; the next runtime on the same (shared) streams
# ---------------------------------------------------------------------------

def _close_then_next_runtime(dev, wait_casts: bool):
    from test1_amd.staging import H2DStager

    comp = dev.default
    h2d, cast = hb_model.FakeStream(dev, "h2d"), hb_model.FakeStream(dev, "cast")
    a = H2DStager("cuda:0", N, 3, h2d, cast, slot_cap_bytes=1 << 30)
    with dev.as_host("update"):
        pc = a.copy_for_later(torch.randn(N), None)
    with dev.as_host("autograd"):
        unit = dev.alloc((N,), torch.bfloat16)
        a.cast_pending(pc, unit, comp)            # reads the slot on the forward's stream
    with dev.as_host("main"):
        # runtime A closes: release_slots drains the copy and cast streams
        h2d.synchronize()
        cast.synchronize()
        dropped = [t for lst in a.slots._free.values() for t, _ in lst]
        if wait_casts:
            a.slots.release(timeout=None)
        else:
            a.slots._free.clear()                 # the release before it waited for the casts
        for t in dropped:
            dev.free(t)                           # the last reference goes
        b = H2DStager("cuda:0", N, 3, h2d, cast, slot_cap_bytes=1 << 30)
    with dev.as_host("update"):
        assert b.copy_for_later(torch.randn(N), None) is not None


def test_slots_released_after_their_last_cast(dev):
    _close_then_next_runtime(dev, wait_casts=True)
    assert dev.races == []


def test_slots_released_before_their_last_cast_race(dev):
    """Without waiting for the casts, the next runtime's copy on the shared
    copy stream reuses a slot's block while the old cast may still read it."""
    _close_then_next_runtime(dev, wait_casts=False)
    assert any("copy on h2d" in r and "cast" in r for r in dev.races), dev.races
