"""Host-side runtime logic that needs no GPU: the buffer pool's blocking and
ordering, and the transfer-strategy factory."""

import threading
import time

import pytest
import torch

import oracle
from test1_amd.layer_state import LayerBufferPool


def test_pool_fifo_and_blocking():
    pool = LayerBufferPool(16, torch.bfloat16, torch.device("cpu"), 2)
    a, b = pool.acquire(), pool.acquire()
    assert a is not b and pool.available() == 0
    got = []
    t = threading.Thread(target=lambda: got.append(pool.acquire(timeout=10)))
    t.start()
    time.sleep(0.2)
    assert not got
    pool.release(a)
    t.join(5)
    assert got and got[0] is a
    with pytest.raises(TimeoutError):
        pool.acquire(timeout=0.05)
    pool.release(b)
    pool.release(a)
    assert pool.acquire() is b  # FIFO order, as the reference's deque


def test_pool_requires_two_units():
    with pytest.raises(ValueError):
        LayerBufferPool(16, torch.bfloat16, torch.device("cpu"), 1)


def test_distributed_sync_factory_single_process():
    from test1_amd import SlideFSDPConfig
    from test1_amd.distributed_sync import NoOpSync, create_distributed_sync

    s = create_distributed_sync(SlideFSDPConfig(device=torch.device("cpu")))
    assert isinstance(s, NoOpSync) and s.world_size == 1 and s.rank == 0


def test_step_schedule_resident_units_drop_backward_loads():
    full = oracle.step_schedule(4, first_decoder_first=True)
    res = oracle.step_schedule(4, first_decoder_first=True, resident_units=(2, 3))
    assert [e for e in full if e not in (("h2d", 2, True), ("h2d", 3, True))] == res
    assert len(full) - len(res) == 2


def test_priority_update_executor_runs_lowest_first_and_reports_errors():
    from test1_amd.layer_state import PriorityUpdateExecutor

    ex = PriorityUpdateExecutor("test-upd")
    gate = threading.Event()
    order = []
    first = ex.submit(0, gate.wait, 10)  # holds the worker while the rest queue up
    futs = [ex.submit(p, order.append, p) for p in (5, 3, 7, 1, 3)]
    bad = ex.submit(4, lambda: 1 / 0)
    gate.set()
    for f in futs:
        f.result(timeout=10)
    assert first.result(timeout=10) is True
    assert order == [1, 3, 3, 5, 7]
    with pytest.raises(ZeroDivisionError):
        bad.result(timeout=10)
    ex.shutdown(wait=True)
    with pytest.raises(RuntimeError):
        ex.submit(0, order.append, 0)


class _FakeReady:
    """Stands in for a copy-completion event; ``synchronize`` completes it."""

    def __init__(self, log, name):
        self.done, self.log, self.name = False, log, name

    def query(self):
        return self.done

    def synchronize(self):
        self.log.append(("waited", self.name))
        self.done = True


def test_priority_update_executor_skips_tasks_whose_input_is_not_ready():
    from test1_amd.layer_state import PriorityUpdateExecutor

    ex = PriorityUpdateExecutor("test-upd2")
    gate = threading.Event()
    log = []
    ex.submit(-1, gate.wait, 10)
    r_old, r_new = _FakeReady(log, "old"), _FakeReady(log, "new")
    ready_mid = _FakeReady(log, "mid")
    ready_mid.done = True
    # priority 1 is not ready: the ready priority-5 task runs first, then the
    # worker waits for the OLDEST pending copy (priority 9), never the newer one
    f9 = ex.submit(9, log.append, 9, ready=r_old)
    f5 = ex.submit(5, log.append, 5, ready=ready_mid)
    f1 = ex.submit(1, log.append, 1, ready=r_new)
    gate.set()
    for f in (f9, f5, f1):
        f.result(timeout=10)
    assert log == [5, ("waited", "old"), 9, ("waited", "new"), 1]
    ex.shutdown(wait=True)


class _PolledReady:
    """Readiness the executor must poll (as a unit whose moments wait for a
    buffer that another queued unit's update frees)."""

    poll_interval = 1e-3
    poll_fallback_s = 30.0

    def __init__(self, cond):
        self.cond = cond

    def query(self):
        return self.cond()

    def synchronize(self):
        raise AssertionError("polled readiness is not waited on")


def test_priority_update_executor_polls_instead_of_committing_to_the_oldest():
    from test1_amd.layer_state import PriorityUpdateExecutor

    ex = PriorityUpdateExecutor("test-upd3")
    gate, flag = threading.Event(), threading.Event()
    log = []
    ex.submit(-1, gate.wait, 10)
    # the oldest task (9) can only become ready after task 5 has run; task 5
    # becomes ready a little later: the worker must wait for 5, run it, then 9
    f9 = ex.submit(9, log.append, 9, ready=_PolledReady(lambda: 5 in log))
    f5 = ex.submit(5, log.append, 5, ready=_PolledReady(flag.is_set))
    gate.set()
    threading.Timer(0.1, flag.set).start()
    for f in (f9, f5):
        f.result(timeout=10)
    assert log == [5, 9]
    # nothing ever ready: after poll_fallback_s the oldest task runs anyway
    never = _PolledReady(lambda: False)
    never.poll_fallback_s = 0.2
    never.synchronize = lambda: None
    f = ex.submit(3, log.append, 3, ready=never)
    f.result(timeout=10)
    assert log == [5, 9, 3]
    ex.shutdown(wait=True)


def test_grad_slots_per_unit_are_sized_and_never_block(monkeypatch):
    from test1_amd import grad_slots
    from test1_amd.grad_slots import GradSlotsPerUnit

    # pinned memory needs a GPU; plain host tensors stand in for it here
    monkeypatch.setattr(grad_slots, "pinned_empty", lambda n, dt: torch.empty(n, dtype=dt))
    slots = GradSlotsPerUnit({0: 10, 1: 0, 2: 7}, torch.bfloat16)
    assert slots.slots[0].numel() == 10 and slots.slots[2].numel() == 7
    assert slots.acquire(timeout=0, unit=2) == 2 and slots.acquire(timeout=0, unit=2) == 2
    slots.release(2)
    with pytest.raises(KeyError):
        slots.acquire(unit=5)


def test_grad_slots_fall_back_to_a_ring_when_pinning_fails(monkeypatch):
    from test1_amd import _native, grad_slots, layer_state

    calls = []

    def fake_pinned(n, dt):
        calls.append(n)
        if len(calls) > 2:  # the host refuses to pin more after two slots
            raise _native.NativeError("sf_host_alloc failed: out of memory", _native.HIP_ERROR_OUT_OF_MEMORY)
        return torch.empty(n, dtype=dt)

    monkeypatch.setattr(grad_slots, "pinned_empty", fake_pinned)
    rt = object.__new__(layer_state.StreamingRuntime)
    rt.grad_ring, rt._dtype, rt.offload_executor, rt.wait_timeout = None, torch.bfloat16, None, None
    rt.pool = type("P", (), {"max_param_size": 9})()
    ring_slots = []
    monkeypatch.setattr(layer_state, "GradSlotRing",
                        lambda sizes, depth, dt: ring_slots.append((dict(sizes), depth)) or
                        type("R", (), {"big": {}, "slot_elems": 9, "acquire": None})())
    rt.init_grad_slots({0: 5, 1: 9, 2: 7, 3: 3})
    assert ring_slots == [({0: 5, 1: 9, 2: 7, 3: 3}, 3)]
    rt.offload_executor.shutdown(wait=True)

    # any other failure is not swallowed
    def broken(n, dt):
        raise _native.NativeError("sf_host_alloc failed: invalid argument", 9001)

    monkeypatch.setattr(grad_slots, "pinned_empty", broken)
    rt.grad_ring = None
    with pytest.raises(_native.NativeError):
        rt.init_grad_slots({0: 5})


def test_gated_executor_gives_the_slot_to_the_most_urgent_ready_task():
    from test1_amd.layer_state import PriorityUpdateExecutor
    import queue as _q

    slots = _q.Queue()
    got = []
    ex = PriorityUpdateExecutor("test-gate", gate=lambda: slots.get(timeout=10))
    # three offloads queue up while no slot is free
    futs = [ex.submit(p, lambda slot, p=p: got.append((p, slot)), ready=None) for p in (30, 10, 20)]
    time.sleep(0.1)
    assert got == []
    for s in ("a", "b", "c"):
        slots.put(s)
    for f in futs:
        f.result(timeout=10)
    assert got == [(10, "a"), (20, "b"), (30, "c")]
    # a gate that fails fails the oldest task, and the worker keeps going
    ex2 = PriorityUpdateExecutor("test-gate2", gate=lambda: (_ for _ in ()).throw(TimeoutError("no slot")))
    f = ex2.submit(1, got.append, 0)
    with pytest.raises(TimeoutError):
        f.result(timeout=10)
    ex2.shutdown(wait=True)
    ex.shutdown(wait=True)


def test_dma_ready_remembers_completion_and_never_queries_freed_signals(monkeypatch):
    """The update executor polls a unit's copies while the update thread may
    free them: once completion has been seen, no query touches the (possibly
    freed) signals again, and they are freed only after completion."""
    from test1_amd import kernels

    state = {"done_after": 3, "queries": 0, "freed": False}

    def fake_query(handle):
        assert not state["freed"], "queried freed signals"
        state["queries"] += 1
        return state["queries"] >= state["done_after"]

    def fake_wait(handle):
        state["freed"] = True
        return (1, 2)

    monkeypatch.setattr(kernels, "dma_query", fake_query)
    monkeypatch.setattr(kernels, "dma_wait", fake_wait)
    r = kernels.DmaReady(("h", 1))
    assert not r.query() and not r.query()
    assert r.release() == (1, 2)          # waits for completion, then frees
    assert state["freed"] and r.query()   # answered from memory
    r.synchronize()
    with pytest.raises(RuntimeError):
        r.release()


def test_grad_slot_ring_gives_big_units_their_own_slot_and_grows(monkeypatch):
    """The fallback when one pinned slot per unit does not fit: units more
    than twice the median size keep their own slot, the rest share a ring of
    slots of the largest remaining unit; ``grow`` pins more ring slots until
    the host refuses, then gives back enough for the headroom."""
    from test1_amd import _native, grad_slots
    from test1_amd.grad_slots import GradSlotRing

    budget = {"left": 10}

    def fake_pinned(n, dt):
        if budget["left"] <= 0:
            raise _native.NativeError("sf_host_alloc failed: out of memory", _native.HIP_ERROR_OUT_OF_MEMORY)
        budget["left"] -= 1
        return torch.empty(n, dtype=dt)

    monkeypatch.setattr(grad_slots, "pinned_empty", fake_pinned)
    sizes = {0: 40, 1: 10, 2: 10, 3: 9, 4: 10, 5: 10, 6: 10, 7: 10, 8: 10, 9: 100}
    ring = GradSlotRing(sizes, 2, torch.bfloat16)
    assert ring.big == {0: 40, 9: 100} and ring.slot_elems == 10 and ring.depth == 2
    assert ring.slots[("unit", 9)].numel() == 100
    assert ring.acquire(unit=9) == ("unit", 9) and ring.own_slot(9) == ("unit", 9) and ring.own_slot(3) is None
    a, b = ring.acquire(timeout=0, unit=3), ring.acquire(timeout=0, unit=4)
    assert {a, b} == {0, 1}
    with pytest.raises(TimeoutError):
        ring.acquire(timeout=0.01, unit=5)
    ring.release(a)
    ring.release(("unit", 9))            # own slots are not ring slots: no-op
    assert ring.acquire(timeout=0, unit=5) == a
    # 6 more allocations succeed, then the host refuses; 2 slots go back as headroom
    added = ring.grow(max_depth=20, headroom_bytes=2 * 10 * 2)
    assert added == 4 and ring.depth == 6
    assert {ring.acquire(timeout=0) for _ in range(4)} == {2, 3, 4, 5}
    # growth stops at max_depth without touching the host limit
    budget["left"] = 100
    assert ring.grow(max_depth=7, headroom_bytes=0) == 1 and ring.depth == 7


def test_save_on_cpu_round_trip():
    """``sliding_checkpoint.save_on_cpu`` (the reference module carries a copy
    of torch's, sliding_checkpoint.py:206-231): saved tensors go to the host
    and come back for the backward."""
    from test1_amd import save_on_cpu

    x = torch.randn(8, 4, requires_grad=True)
    with save_on_cpu(pin_memory=False):
        y = (x * x).sum()
    y.backward()
    assert torch.allclose(x.grad, 2 * x.detach())


@pytest.mark.parametrize("args,env", [(["--gpus", "2"], {}), (["--gpus", "1"], {"WORLD_SIZE": "2"})])
def test_bench_refuses_more_than_one_gpu(args, env):
    """The path runs on one GPU: bench.py with --gpus above 1, or launched as
    one of several ranks, exits with status 2 and says so, before touching a
    GPU."""
    import os
    import subprocess
    import sys

    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    r = subprocess.run([sys.executable, os.path.join(root, "bench.py")] + args, capture_output=True, text=True,
                       env={**os.environ, **env}, timeout=120)
    assert r.returncode == 2, (r.returncode, r.stderr[-500:])
    assert "one GPU only" in r.stderr


def test_copy_backlog_trims_safely_from_several_threads():
    """The copy backlog is trimmed by several threads at once while another
    appends: no event is lost or popped twice, and the count ends at the
    events still pending."""
    import threading
    from collections import deque

    from test1_amd.layer_state import _backlog

    class Ev:
        def __init__(self, done):
            self.done = done

        def query(self):
            return self.done

    copies = deque(Ev(True) for _ in range(20000))
    errors = []

    def trim():
        try:
            for _ in range(2000):
                _backlog(copies)
        except BaseException as e:  # noqa: BLE001 - the test reports any failure
            errors.append(e)

    ts = [threading.Thread(target=trim) for _ in range(4)]
    for t in ts:
        t.start()
    for _ in range(5000):
        copies.append(Ev(True))
    for t in ts:
        t.join()
    copies.append(Ev(False))
    copies.append(Ev(True))
    assert not errors
    assert _backlog(copies) == 2


def test_priority_update_executor_survives_a_failing_readiness_query():
    """A task whose readiness query raises is run (and reports its own
    error) instead of stopping the worker thread; later tasks still run."""
    from test1_amd.layer_state import PriorityUpdateExecutor

    class Broken:
        def query(self):
            raise RuntimeError("event lost")

        def synchronize(self):
            raise RuntimeError("event lost")

    ex = PriorityUpdateExecutor("test-exec")
    try:
        def boom():
            raise ValueError("input failed")

        f1 = ex.submit(0, boom, ready=Broken())
        f2 = ex.submit(1, lambda: 42)
        with pytest.raises(ValueError):
            f1.result(timeout=10)
        assert f2.result(timeout=10) == 42
    finally:
        ex.shutdown()


def test_bench_link_arithmetic():
    """The bench's host-link figures: transfers of one direction that overlap
    count their bytes once over the union of their intervals, and the share
    under compute is the intersection of that union with the compute
    intervals."""
    import bench

    assert bench._union([(5, 7, 0), (0, 2, 0), (1, 3, 0), (7, 8, 0)]) == [[0, 3], [5, 8]]
    assert bench._overlap([[0, 3], [5, 8]], [[2, 6], [7, 100]]) == 1 + 1 + 1
    ms = 1_000_000   # ns
    r = {"elapsed": 0.1, "link": {
        "h2d": {"params": [(0, 20 * ms, 1_000_000_000)], "checkpoints": [(10 * ms, 30 * ms, 500_000_000)],
                "rows": []},
        "d2h": {"grads": [(40 * ms, 50 * ms, 400_000_000)], "checkpoints": [], "rows": []},
        "compute": [(0, 15 * ms), (45 * ms, 60 * ms)],
        "common_clock": True}}
    st = bench.link_stats(r, steps=1, alone={"h2d_gbs": 60.0, "d2h_gbs": 50.0})
    h = st["h2d"]
    assert h["busy_ms_per_step"] == 30 and h["bytes_per_step"] == 1.5e9
    assert abs(h["gbs_while_busy"] - 50.0) < 1e-9 and abs(h["frac_of_measured_copy"] - 50 / 60) < 1e-9
    assert abs(h["under_compute_frac"] - 0.5) < 1e-9          # 15 of 30 ms under compute
    d = st["d2h"]
    assert abs(d["gbs_while_busy"] - 40.0) < 1e-9 and abs(d["under_compute_frac"] - 0.5) < 1e-9
    assert abs(st["compute_busy_frac_of_step"] - 0.3) < 1e-9
    r["link"]["common_clock"] = False                          # no SDMA clock: no overlap figure
    assert bench.link_stats(r, steps=1)["h2d"]["under_compute_frac"] is None
    assert "untimed_bytes_per_step" not in st["d2h"]
    # gradient copies without engine timestamps are reported, not counted as 0 B
    r["link"]["untimed_d2h_bytes"] = 600_000_000
    d = bench.link_stats(r, steps=2)["d2h"]
    assert d["untimed_bytes_per_step"] == 3e8 and d["bytes_per_step_by_kind"]["grads"] == 2e8
    recs = [("untimed", 600_000_000), ("interval_ns", 0, 10 * ms, 400_000_000)]
    assert bench.elapsed_stats(recs) == (10.0, 400_000_000)


def test_bench_copy_model_and_h2d_idle_attribution():
    """``frac_of_copy_model``: bytes over what plain copies move in the same
    busy time, at the duplex rate while the other direction is busy and the
    one-way rate otherwise.  ``h2d_idle_attribution``: each H2D gap goes to
    what the copy ending it waited for (issued under 1 ms before it started:
    the thread that issued it; earlier: the device)."""
    import bench

    ms = 1_000_000   # ns
    # H2D busy [0, 10] ms, D2H busy [5, 20] ms: 5 ms duplex, 5 ms one way for H2D
    alone = {"h2d_gbs": 50.0, "d2h_gbs": 56.0, "duplex": {"h2d_gbs": 40.0, "d2h_gbs": 52.0}}
    r = {"elapsed": 0.02, "link": {
        "h2d": {"params": [(0, 10 * ms, 450_000_000)], "checkpoints": [], "rows": []},
        "d2h": {"grads": [(5 * ms, 20 * ms, 700_000_000)], "checkpoints": [], "rows": []},
        "compute": [], "common_clock": True}}
    st = bench.link_stats(r, steps=1, alone=alone)
    # H2D: 5 ms x 40 GB/s + 5 ms x 50 GB/s = 450 MB; D2H: 5 x 52 + 10 x 56 = 820 MB
    assert abs(st["h2d"]["frac_of_copy_model"] - 1.0) < 1e-12
    assert abs(st["d2h"]["frac_of_copy_model"] - 700 / 820) < 1e-12
    assert st["h2d"]["both_directions_busy_ms_per_step"] == 5
    assert abs(st["h2d"]["frac_of_duplex_copy"] - 45 / 40) < 1e-12
    assert bench.link_stats(r, steps=1, alone={"h2d_gbs": 50.0})["h2d"]["frac_of_copy_model"] is None

    # H2D copies (ms on the host timeline's clock) [2, 4], [6, 8], [8.5, 9.5] in a 12 ms window
    anchor = 1_000 * ms
    link = {"h2d": {"params": [(anchor + 2 * ms, anchor + 4 * ms, 1), (anchor + 6 * ms, anchor + 8 * ms, 1)],
                    "checkpoints": [(anchor + int(8.5 * ms), anchor + int(9.5 * ms), 1)], "rows": []}}
    events = [(0.0015, "sf-update", "staged_after_update", 3),     # 1.5 ms: issued 0.5 ms before its copy
              (0.0030, "MainThread", "h2d_issued", 4),             # 3 ms: 3 ms before the copy at 6 ms
              (0.0082, "MainThread", "h2d_issued", 5)]             # 8.2 ms: 0.3 ms before the one at 8.5
    out = bench.h2d_idle_attribution(events, link, anchor, 0.012)
    assert out["gaps"] == 4 and abs(out["idle_ms"] - (2 + 2 + 0.5 + 2.5)) < 1e-9
    assert abs(out["waiting_for_update_thread_ms"] - 2) < 1e-9        # [0, 2] ended by unit 3's copy
    assert abs(out["waiting_on_device_ms"] - 2) < 1e-9                # [4, 6]: issued at 3 ms
    assert abs(out["waiting_for_forward_ms"] - 0.5) < 1e-9            # [8, 8.5]
    assert abs(out["idle_frac"] - 7 / 12) < 1e-9                       # the tail [9.5, 12] is idle, unattributed


def test_checkpoint_slot_kept_on_device_only_when_pinning_runs_out(monkeypatch):
    """A checkpoint slot the host cannot pin (out of memory) becomes a
    ``KeptOnDevice`` marker of the slot's shape and dtype; any other failure
    of the pinned allocation still raises."""
    from test1_amd import _native, sliding_checkpoint as sc

    def refuse(status):
        def pinned_empty(shape, dtype):
            raise _native.NativeError("sf_host_alloc failed", status)
        return pinned_empty

    monkeypatch.setattr(sc, "pinned_empty", refuse(_native.HIP_ERROR_OUT_OF_MEMORY))
    kept = sc.pin_or_keep((4, 16, 32), torch.bfloat16)
    assert isinstance(kept, sc.KeptOnDevice)
    assert kept.shape == (4, 16, 32) and kept.dtype == torch.bfloat16
    monkeypatch.setattr(sc, "pinned_empty", refuse(1))
    with pytest.raises(_native.NativeError):
        sc.pin_or_keep((4, 16, 32), torch.bfloat16)


def test_bench_host_dram_counts_every_host_link_transfer():
    """``host_dram``: the AdamW's 26 B per parameter (28 with bf16 H2D) plus
    every host-link transfer of the timed steps, gradient copies without
    engine timestamps included; without link records, the copy totals."""
    from types import SimpleNamespace

    import bench

    r = {"total_params": 1000, "elapsed": 2.0, "h2d": (1.0, 4000), "d2h": (1.0, 2000), "link": {
        "h2d": {"params": [(0, 1, 4000)], "checkpoints": [(0, 1, 300)], "rows": [(0, 1, 50)]},
        "d2h": {"grads": [(0, 1, 1500)], "checkpoints": [(0, 1, 300)], "rows": [(0, 1, 25)]},
        "untimed_d2h_bytes": 500}}
    args = SimpleNamespace(h2d_format="fp32", steps=2)
    st = bench.host_dram_stats(r, args, {"adam_gbs": 1e-5})
    assert st["adam_bytes_per_step"] == 26_000
    assert st["bytes_per_step"] == 26_000 + (4000 + 300 + 50 + 1500 + 300 + 25 + 500) / 2
    assert abs(st["achieved_gbs"] - st["bytes_per_step"] / 1.0 / 1e9) < 1e-18
    assert abs(st["frac_of_streaming_adam"] - st["achieved_gbs"] / 1e-5) < 1e-9
    r["link"] = {}
    st = bench.host_dram_stats(r, SimpleNamespace(h2d_format="bf16", steps=2), None)
    assert st["bytes_per_step"] == 28_000 + 3000 and st["frac_of_streaming_adam"] is None


@pytest.mark.parametrize("adam,omp,cores,expected", [
    (None, None, 16, 15), ("", "", 16, 15), ("0", None, 16, 15), ("12", None, 16, 12), (" 4 ", "2", 16, 4),
    (None, "8", 16, 7), (None, "8,2", 16, 7), (None, "32", 16, 15), (None, "x", 16, 15), (None, "1", 16, 1),
    (None, None, 1, 1)])
def test_adam_threads_from_the_environment(monkeypatch, adam, omp, cores, expected):
    from test1_amd import slide_fsdp
    for name, value in (("SF_ADAM_THREADS", adam), ("OMP_NUM_THREADS", omp)):
        if value is None:
            monkeypatch.delenv(name, raising=False)
        else:
            monkeypatch.setenv(name, value)
    monkeypatch.setattr(slide_fsdp, "_cpu_count", lambda: cores)
    assert slide_fsdp.adam_threads() == expected


@pytest.mark.parametrize("adam", ["-2", "four", "2.5"])
def test_adam_threads_rejects_other_values(monkeypatch, adam):
    from test1_amd import slide_fsdp
    monkeypatch.setenv("SF_ADAM_THREADS", adam)
    with pytest.raises(ValueError, match="SF_ADAM_THREADS"):
        slide_fsdp.adam_threads()
