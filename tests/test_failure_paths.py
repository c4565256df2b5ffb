"""Failure handling of the runtime, on the CPU with stand-ins for the device
parts: a gradient offload whose SDMA copies fail part-way never hands its
host slot back while a copy may still write into it, bounded waits raise
TimeoutError naming the unit, an aborted piecewise staging keeps its slot's
fence, and an early embedding update left without its late part (the
backward failed) is cancelled or completed consistently."""

import threading
import time

import pytest
import torch

from test1_amd import _native, kernels


# ---------------------------------------------------------------------------
# SDMA copies that fail after some were issued (kernels level)
# ---------------------------------------------------------------------------

class _StubHip:
    """sf_dma_* entry points: ``copy`` fails after issuing two copies, which
    complete after ``polls_to_done`` queries (never, if None)."""

    def __init__(self, polls_to_done):
        self.polls_to_done = polls_to_done
        self.queries = 0
        self.waited = []

    def sf_dma_query(self, handles, n, done):
        self.queries += 1
        done._obj.value = int(self.polls_to_done is not None and self.queries >= self.polls_to_done)
        return 0

    def sf_dma_wait(self, handles, n, timeout_ns, t0, t1):
        if self.polls_to_done is None and timeout_ns:
            return _native.SF_ETIMEDOUT       # still pending at the deadline: nothing released
        self.waited.append([handles[i] for i in range(n)])
        return 0

    def sf_error_string(self, status):
        return b"sf: too many segments for one call"


def test_failed_issue_waits_for_the_copies_it_started(monkeypatch):
    stub = _StubHip(polls_to_done=3)
    monkeypatch.setattr(_native, "hip", lambda: stub)
    handles = (kernels.ctypes.c_uint64 * 4)(11, 12, 0, 0)
    with pytest.raises(_native.NativeError) as e:
        kernels._issued_or_raise(9002, handles, 2, timeout=5.0)
    assert e.value.status == 9002
    assert stub.queries == 3 and stub.waited == [[11, 12]]   # completed and released before the raise


def test_failed_issue_with_copies_that_never_land(monkeypatch):
    stub = _StubHip(polls_to_done=None)
    monkeypatch.setattr(_native, "hip", lambda: stub)
    handles = (kernels.ctypes.c_uint64 * 2)(11, 12)
    t = time.monotonic()
    with pytest.raises(kernels.DmaCopiesOutstanding):
        kernels._issued_or_raise(9002, handles, 2, timeout=0.05)
    assert time.monotonic() - t < 2.0 and stub.waited == []   # never released: still in flight


def test_dma_ready_wait_is_bounded(monkeypatch):
    stub = _StubHip(polls_to_done=None)
    monkeypatch.setattr(_native, "hip", lambda: stub)
    handles = (kernels.ctypes.c_uint64 * 1)(7)
    r = kernels.DmaReady((handles, 1), timeout=0.05)
    with pytest.raises(kernels.DmaCopiesOutstanding):
        r.release()
    assert stub.waited == []


def test_dma_wait_deadline_keeps_the_copies(monkeypatch):
    stub = _StubHip(polls_to_done=None)
    monkeypatch.setattr(_native, "hip", lambda: stub)
    handles = (kernels.ctypes.c_uint64 * 2)(5, 6)
    with pytest.raises(kernels.DmaCopiesOutstanding):
        kernels.dma_wait((handles, 2), timeout=0.01)
    assert stub.waited == []


def test_wait_event_is_bounded():
    class Never:
        def query(self):
            return False

    with pytest.raises(TimeoutError, match="unit 7: gradients"):
        kernels.wait_event(Never(), 0.05, "unit 7: gradients")


# ---------------------------------------------------------------------------
# Gradient offload task: copies of the first piece issued, the second fails
# ---------------------------------------------------------------------------

class _Event:
    def query(self):
        return True

    def synchronize(self):
        pass


class _Ring:
    def __init__(self, n):
        self.slots = {0: torch.zeros(n, dtype=torch.bfloat16)}
        self.released = []

    def release(self, idx):
        self.released.append(idx)


class _Runtime:
    def __init__(self, n):
        self.grad_ring = _Ring(n)
        self.wait_timeout = 0.2
        self.d2h_engine = "sdma"
        self.held = []

    def mark(self, *a):
        pass

    def hold_forever(self, objs):
        self.held.append(objs)


def _offload_state(monkeypatch, copies_land):
    """A LayerRuntimeState reduced to what ``_d2h_task`` touches, updated in
    two pieces; the second piece's copy fails to issue."""
    from test1_amd import layer_state

    order = []
    st = object.__new__(layer_state.LayerRuntimeState)
    st.__dict__.update(runtime=_Runtime(16), layer_idx=3, update_finished=threading.Event())
    st._piece_plan = lambda: ([(0, 8), (8, 16)], None)

    def copy(pairs, timeout=None):
        if order.count("issue") == 1:
            raise _native.NativeError("sf_dma_copy_d2h failed: ROCr DMA call failed", 10001)
        order.append("issue")
        return ("handle", len(pairs))

    class Ready:
        def __init__(self, handle, timeout=None):
            self.handle = handle

        def release(self):
            if not copies_land:
                raise kernels.DmaCopiesOutstanding("1 SDMA copy not complete")
            order.append("landed")
            return (0, 0)

    monkeypatch.setattr(kernels, "dma_copy_d2h", copy)
    monkeypatch.setattr(kernels, "DmaReady", Ready)
    return st, order


def test_offload_failure_releases_the_slot_after_its_copies_land(monkeypatch):
    st, order = _offload_state(monkeypatch, copies_land=True)
    st.runtime.grad_ring.release = lambda idx: order.append(("slot released", idx))
    grads = [(torch.zeros(16, dtype=torch.bfloat16), 0)]
    with pytest.raises(_native.NativeError):
        st._d2h_task(0, grads, [], _Event(), None)
    assert order == ["issue", "landed", ("slot released", 0)]
    assert st.update_finished.is_set() and st.runtime.held == []


def test_offload_failure_keeps_the_slot_while_a_copy_is_outstanding(monkeypatch):
    st, order = _offload_state(monkeypatch, copies_land=False)
    grads = [(torch.zeros(16, dtype=torch.bfloat16), 0)]
    with pytest.raises(_native.NativeError):
        st._d2h_task(0, grads, [], _Event(), None)
    assert st.runtime.grad_ring.released == []           # an engine may still write into it
    (held_grads, issued, slot), = st.runtime.held        # sources and slot kept for good
    assert slot == 0 and held_grads is grads and issued == [("handle", 1)]
    assert st.update_finished.is_set()


def test_update_wait_timeout_names_the_unit():
    from concurrent.futures import Future

    from test1_amd import layer_state

    st = object.__new__(layer_state.LayerRuntimeState)
    rt = _Runtime(1)
    st.__dict__.update(runtime=rt, layer_idx=5, update_finished=threading.Event(),
                       _d2h_future=None, _update_future=Future())
    with pytest.raises(TimeoutError, match="Layer 5 parameter update not finished"):
        st.wait_for_update(timeout=0.05)


def test_executor_shutdown_is_bounded():
    from test1_amd.update_executor import PriorityUpdateExecutor

    gate = threading.Event()
    ex = PriorityUpdateExecutor("sf-test")
    ex.submit(0, gate.wait)
    time.sleep(0.05)
    with pytest.raises(TimeoutError, match="sf-test"):
        ex.shutdown(wait=True, timeout=0.1)
    gate.set()
    ex.shutdown(wait=True, timeout=5)


# ---------------------------------------------------------------------------
# Piecewise staging aborted before its first piece
# ---------------------------------------------------------------------------

def test_aborted_pieces_keep_the_slot_fence():
    from test1_amd.staging import _StagerPieces

    given = []

    class Slots:
        def give(self, t, ev):
            given.append((t, ev))

    stager = type("S", (), {"slots": Slots()})()
    buf, fence = torch.empty(10), object()
    p = _StagerPieces(stager, torch.zeros(10), torch.empty(10), None, [(0, 4), (4, 10)], (buf, fence))
    p.abort()
    assert given == [(buf, fence)]       # the next copy into the slot still waits for its last reader
    p2 = _StagerPieces(stager, torch.zeros(10), torch.empty(10), None, [(0, 4), (4, 10)], (buf, fence))
    p2.pushed, p2.last_issued = 1, "copy event"
    p2.abort()
    assert given[-1] == (buf, "copy event")


# ---------------------------------------------------------------------------
# Early embedding update whose backward failed
# ---------------------------------------------------------------------------

V, H = 64, 32


def _embedding_state(seed=0):
    """A row-sparse embedding unit on the host: a real LayerAdam (reference
    order) and a real update thread; the device parts are stand-ins."""
    from test1_amd import layer_state
    from test1_amd.optimizer import LayerAdam
    from test1_amd.update_executor import PriorityUpdateExecutor

    table = torch.nn.Parameter(torch.randn(V, H, generator=torch.Generator().manual_seed(seed)) * 0.02)
    opt = LayerAdam(lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.01, num_layer=1)
    opt.reference_order = True
    opt.add_layer_params(0, [table])
    st = object.__new__(layer_state.LayerRuntimeState)
    rt = type("RT", (), {})()
    rt.wait_timeout = 10.0
    rt.capturing = lambda u: False
    rt.mark = lambda *a: None
    rt.set_adam_threads = lambda: None
    rt.update_executor = PriorityUpdateExecutor("sf-update-test")
    st.__dict__.update(runtime=rt, layer_idx=0, layer_optimizer=opt, _rows_shape=(V, H),
                       _cpu_params_flat=table.data.view(-1), _cpu_params_bf16=None,
                       update_lock=threading.Lock(), _early_lock=threading.Lock(), _early=None)
    return st, opt, table


def _queue_early(st, ids):
    early = {"ids": ids, "ready": _Event(), "state": "queued"}
    st._early = early
    early["future"] = st.runtime.update_executor.submit(1 << 30, st._do_update_rows_early, early)
    return early


def test_orphaned_early_update_that_ran_is_completed_with_zero_gradient():
    ids = torch.tensor([3, 9, 40, 41])
    st, opt, table = _embedding_state()
    early = _queue_early(st, ids)
    early["future"].result(timeout=10)
    assert early["state"] == "applied"
    st.settle_orphaned_early()
    assert st._early is None and opt._early_rows == {}
    # the same as one whole step of the table with a zero gradient everywhere
    ref_st, ref_opt, ref_table = _embedding_state()
    with torch.no_grad():
        ref_opt.step_rows(0, torch.full((V,), _native.SF_ROW_ZERO, dtype=torch.int64),
                          torch.empty((0, H), dtype=torch.bfloat16), ref_table.data)
    assert torch.equal(table.data.view(torch.int32), ref_table.data.view(torch.int32))
    assert opt.param_groups[0]["step"] == ref_opt.param_groups[0]["step"] == 1
    for ex in (st.runtime.update_executor, ref_st.runtime.update_executor):
        ex.shutdown(timeout=5)


def test_orphaned_early_update_still_queued_is_cancelled():
    st, opt, table = _embedding_state()
    before = table.data.clone()
    gate = threading.Event()
    st.runtime.update_executor.submit(0, gate.wait)      # keeps the worker busy
    early = _queue_early(st, torch.tensor([1, 2]))
    st.settle_orphaned_early()
    assert early["state"] == "cancelled"
    gate.set()
    st.runtime.update_executor.shutdown(timeout=5)       # runs whatever is left queued
    assert torch.equal(table.data, before)                # the table never moved
    assert opt.param_groups[0]["step"] == 0 and opt._early_rows == {}
