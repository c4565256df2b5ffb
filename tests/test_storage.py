"""Storage offload: the native file engine, the moment offloader and
LayerAdam's NVMe offload, on the host.

What the offload must preserve is identity: bytes written come back
unchanged, and training with moments on storage gives the bits of training
with moments in memory (which the LayerAdam tests pin against the reference's
compiled cpu_adam).  The reference's tensornvme / kvikio back ends are not
installed anywhere here, so their own behaviour is not compared."""

import random

import pytest
import torch

from test1_amd import _native, storage
from test1_amd.optimizer import LayerAdam, cpu_adam
from test1_amd.optimizer.state_offload import StateOffloader


@pytest.fixture(autouse=True)
def _threads():
    cpu_adam.set_num_threads(4)
    yield
    cpu_adam.set_num_threads(0)


@pytest.fixture(scope="module")
def engine():
    e = storage.IoEngine(n_threads=4, chunk_bytes=64 << 10)
    yield e
    e.close()


def test_abi_exports_io_entry_points():
    lib = _native.cpu()
    for name in ("sf_io_create", "sf_io_destroy", "sf_io_open", "sf_io_reserve", "sf_io_close",
                 "sf_io_submit", "sf_io_query", "sf_io_wait", "sf_io_stats"):
        assert hasattr(lib, name)


@pytest.mark.parametrize("direct", [True, False])
def test_round_trip_and_zero_reads(engine, tmp_path, direct):
    f = engine.open(str(tmp_path / "a.bin"), direct=direct)
    n = (3 << 20) // 4  # 3 MiB: many 64 KiB chunks on 4 workers
    a = storage.aligned_empty(n)
    a.copy_(torch.randn(n, generator=torch.Generator().manual_seed(0)))
    f.reserve(4 * n * 3)
    f.write(a, 4 * n).wait()
    b = storage.aligned_empty(n)
    f.read(b, 4 * n).wait()
    assert torch.equal(a.view(torch.int32), b.view(torch.int32))
    z = storage.aligned_empty(n).fill_(7.0)
    f.read(z, 0).wait()          # reserved, never written: zeros
    assert bool((z == 0).all())
    f.close()


def test_many_requests_in_flight_match_a_byte_model(engine, tmp_path):
    """Random writes and reads of 4 KiB-aligned ranges, several in flight at
    once (disjoint ranges), checked against an in-memory copy of the file."""
    rng = random.Random(3)
    f = engine.open(str(tmp_path / "m.bin"))
    blocks = 256
    f.reserve(blocks * 4096)
    model = torch.zeros(blocks * 4096, dtype=torch.uint8)
    for _ in range(20):
        starts = rng.sample(range(0, blocks, 8), 6)
        reqs, bufs = [], []
        for s in starts:
            nb = rng.randint(1, 8)
            buf = storage.aligned_empty(nb * 4096, torch.uint8)
            if rng.random() < 0.5:
                buf.copy_(torch.randint(0, 256, (nb * 4096,), dtype=torch.uint8))
                model[s * 4096:(s + nb) * 4096] = buf
                reqs.append(f.write(buf, s * 4096))
            else:
                reqs.append(f.read(buf, s * 4096))
                bufs.append((buf, s, nb))
        for r in reqs:
            r.wait()
        for buf, s, nb in bufs:
            assert torch.equal(buf, model[s * 4096:(s + nb) * 4096])
    whole = storage.aligned_empty(blocks * 4096, torch.uint8)
    f.read(whole, 0).wait()
    assert torch.equal(whole, model)
    f.close()


def test_alignment_and_errors(engine, tmp_path):
    f = engine.open(str(tmp_path / "e.bin"), direct=True)
    if not f.direct:
        pytest.skip("file system without O_DIRECT")
    a = storage.aligned_empty(4096)
    f.reserve(1 << 20)
    with pytest.raises(_native.NativeError) as ei:
        f.read(a[1:], 0)                                 # unaligned address
    assert ei.value.status == _native.SF_EALIGN
    with pytest.raises(_native.NativeError):
        f.write(a, 100)                                  # unaligned offset
    with pytest.raises(_native.NativeError):
        f.write(a, 0, nbytes=1000)                       # unaligned size
    r = f.read(a, 1 << 20)                               # past the end: ENODATA when waited
    with pytest.raises(_native.NativeError):
        r.wait()
    f.close()
    # unknown ticket, and a second wait of a released one
    lib = _native.cpu()
    assert lib.sf_io_wait(engine.handle, 10 ** 12, None, None) == 9006
    with pytest.raises(_native.NativeError):
        storage.IoEngine(n_threads=0)


def test_stats_count_bytes(tmp_path):
    e = storage.IoEngine(n_threads=2)
    f = e.open(str(tmp_path / "s.bin"))
    a = storage.aligned_empty(1 << 18)
    f.reserve(2 << 20)
    f.write(a, 0).wait()
    f.read(a, 0).wait()
    f.read(a, 1 << 20).wait()
    st = e.stats()
    assert st["bytes_written"] == 1 << 20 and st["bytes_read"] == 2 << 20 and st["busy_s"] > 0
    f.close()
    e.close()


@pytest.mark.parametrize("n_buffers", [2, 3])
def test_offloader_matches_a_dict_model(engine, tmp_path, n_buffers):
    """Units of different sizes acquired, changed and released in random order
    with random prefetches: every acquire sees exactly what the last release
    of that unit left, and untouched units read as zeros."""
    rng = random.Random(n_buffers)
    off = StateOffloader(str(tmp_path), n_moments=2, n_buffers=n_buffers, engine=engine)
    sizes = {u: rng.choice([1000, 4096, 5003, 20000]) for u in range(7)}
    for u, n in sizes.items():
        off.register(u, n)
    model = {u: [torch.zeros(n), torch.zeros(n)] for u, n in sizes.items()}
    for it in range(60):
        for u in rng.sample(list(sizes), rng.randint(0, 3)):
            off.prefetch(u, priority=rng.random())
        u = rng.choice(list(sizes))
        m, v = off.acquire(u)
        assert m.numel() == sizes[u] and v.numel() == sizes[u]
        assert torch.equal(m, model[u][0]) and torch.equal(v, model[u][1]), (it, u)
        m.add_(torch.randn(sizes[u]))
        v.mul_(0.5).add_(1.0)
        model[u] = [m.clone(), v.clone()]
        off.release(u, dirty=True)
    off.flush()
    for u in sizes:
        m, v = off.read_back(u)
        assert torch.equal(m, model[u][0]) and torch.equal(v, model[u][1])
    assert len(off._buffers) <= n_buffers
    off.close()


@pytest.mark.parametrize("n_buffers", [2, 3])
def test_every_requested_unit_becomes_ready(engine, tmp_path, n_buffers):
    """A scheduler that updates only units whose moments are ready (as the
    update thread does) must never starve: units requested while their
    moments are still cached from their last update keep that buffer, and
    requested units without a buffer are read as buffers drain.  (A cached
    unit once lost its buffer to another unit's read and was then never read
    back, so a poll-until-ready scheduler waited forever.)"""
    off = StateOffloader(str(tmp_path), n_moments=1, n_buffers=n_buffers, engine=engine)
    n_units = 6
    for u in range(n_units):
        off.register(u, 3000 + 100 * u)
    rng = random.Random(n_buffers)
    vals = {u: 0.0 for u in range(n_units)}
    for step in range(5):
        order = list(range(n_units))
        rng.shuffle(order)
        for pri, u in enumerate(order):       # requests arrive while earlier units update
            off.prefetch(u, priority=rng.random())
        remaining = set(order)
        for _ in range(20000):
            if not remaining:
                break
            for u in sorted(remaining):
                if off.ready(u):
                    (m,) = off.acquire(u)
                    assert bool((m == vals[u]).all()), (step, u)
                    m.add_(1.0)
                    vals[u] += 1.0
                    off.release(u)
                    remaining.discard(u)
                    break
            else:
                import time
                time.sleep(1e-4)
        assert not remaining, f"step {step}: units {sorted(remaining)} never became ready"
    off.close()


def _units(seed, sizes):
    g = torch.Generator().manual_seed(seed)
    return {u: [torch.nn.Parameter(torch.randn(s, generator=g) * 0.02) for s in shp] for u, shp in sizes.items()}


@pytest.mark.parametrize("fraction", [0.3, 0.8])
@pytest.mark.parametrize("order", ["descending", "shuffled_with_hints"])
def test_layer_adam_offload_is_bit_identical(tmp_path, fraction, order):
    """Several steps over 5 units: moments on storage (2 buffers, so units
    are evicted and read back every step) give the params and moments of
    moments in memory, bit for bit."""
    sizes = {0: [(64, 16)], 1: [(48, 32), (32,)], 2: [(96, 40), (40,), (40,)], 3: [(33, 17)], 4: [(128, 8)]}
    ref_units, off_units = _units(1, sizes), _units(1, sizes)
    kw = dict(lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.01, num_layer=len(sizes))
    ref = LayerAdam(**kw)
    off = LayerAdam(**kw, nvme_offload_fraction=fraction, offload_dir=str(tmp_path), nvme_buffers=2)
    for u in sizes:
        ref.add_layer_params(u, ref_units[u])
        off.add_layer_params(u, off_units[u])
    assert off.exp_avg_flat[0].numel() == 0
    assert (off.exp_avg_sq_flat[0].numel() == 0) == (fraction > 0.5)
    rng = random.Random(5)
    g = torch.Generator().manual_seed(9)
    for step in range(4):
        units = sorted(sizes, reverse=True)
        if order != "descending":
            rng.shuffle(units)
            for pri, u in enumerate(units):
                off.prefetch_states(u, priority=pri)
        for u in units:
            grads = {}
            for pr, po in zip(ref_units[u], off_units[u]):
                gr = (torch.randn(pr.shape, generator=g) * 1e-3).bfloat16()
                grads[pr], grads[po] = gr, gr.clone()
            ref.step_with_grad_views(u, {p: grads[p] for p in ref_units[u]})
            off.step_with_grad_views(u, {p: grads[p] for p in off_units[u]})
    for u in sizes:
        for pr, po in zip(ref_units[u], off_units[u]):
            assert torch.equal(pr.data.view(torch.int32), po.data.view(torch.int32)), u
        rm, rv = ref.layer_states(u)
        om, ov = off.layer_states(u)
        assert torch.equal(rm.view(torch.int32), om.view(torch.int32))
        assert torch.equal(rv.view(torch.int32), ov.view(torch.int32))
        assert off.state[off_units[u][0]]["exp_avg"].numel() == 0   # nothing held between steps
    with pytest.raises(RuntimeError):
        off.step(None)


def test_layer_adam_offload_row_sparse_update(tmp_path):
    """The row-sparse update of an offloaded table equals the in-memory one."""
    V, H = 64, 16
    g = torch.Generator().manual_seed(2)
    w0 = torch.randn(V, H, generator=g) * 0.02
    pr, po = torch.nn.Parameter(w0.clone()), torch.nn.Parameter(w0.clone())
    kw = dict(lr=1e-3, weight_decay=0.01, num_layer=1)
    ref = LayerAdam(**kw)
    off = LayerAdam(**kw, nvme_offload_fraction=1.0, offload_dir=str(tmp_path), nvme_buffers=2)
    ref.add_layer_params(0, [pr])
    off.add_layer_params(0, [po])
    for _ in range(3):
        ids = torch.randint(0, V, (10,), generator=g).unique()
        row_slot = torch.full((V,), -1, dtype=torch.int64)
        row_slot[ids] = torch.arange(ids.numel())
        rows = (torch.randn(ids.numel(), H, generator=g) * 1e-3).bfloat16()
        ref.step_rows(0, row_slot, rows, pr.data)
        off.step_rows(0, row_slot, rows.clone(), po.data)
    assert torch.equal(pr.data.view(torch.int32), po.data.view(torch.int32))
    for a, b in zip(ref.layer_states(0), off.layer_states(0)):
        assert torch.equal(a.view(torch.int32), b.view(torch.int32))


@pytest.mark.parametrize("value", ["0", "-1", "many"])
def test_io_threads_env_rejects_other_values(monkeypatch, value):
    from test1_amd import storage
    monkeypatch.setattr(storage, "_default", None)
    monkeypatch.setenv("SF_IO_THREADS", value)
    with pytest.raises(ValueError, match="SF_IO_THREADS"):
        storage.default_engine()


class _FakeDma:
    """Stands in for the SDMA copy of ``StorageSpill.write_after_dma`` on the
    CPU: copies at once; ``release`` returns engine times or raises."""

    def __init__(self, stuck):
        self.stuck = stuck

    def copy(self, pairs, timeout=None):
        for src, dst in pairs:
            dst.copy_(src.view(torch.uint8).reshape(-1))
        return "handle"

    def ready(self, handle, timeout=None):
        fake = self

        class Ready:
            def release(self):
                if fake.stuck:
                    raise kernels_mod().DmaCopiesOutstanding("1 SDMA copies not complete")
                return 10, 20
        return Ready()


def kernels_mod():
    from test1_amd import kernels
    return kernels


def _spill_with_fake_dma(monkeypatch, tmp_path, stuck):
    from test1_amd import sliding_checkpoint as sc

    fake = _FakeDma(stuck)
    k = kernels_mod()
    monkeypatch.setattr(k, "wait_event", lambda ev, timeout, what: None)
    monkeypatch.setattr(k, "dma_copy_d2h", fake.copy)
    monkeypatch.setattr(k, "DmaReady", fake.ready)
    spill = sc.StorageSpill(n_slots=2, engine=storage.IoEngine(n_threads=2), direct=False)
    slot = object.__new__(sc._BounceSlot)
    slot.buf, slot.held, slot.pending = torch.zeros(storage.align_up(4096), dtype=torch.uint8), True, []
    return spill, slot


def test_checkpoint_to_storage_by_sdma_copy(monkeypatch, tmp_path):
    """The spill's worker waits for the producer, copies into the bounce
    slot, records the copy's engine times, then writes the file; the slot is
    free again after the write."""
    spill, slot = _spill_with_fake_dma(monkeypatch, tmp_path, stuck=False)
    src = torch.arange(2048, dtype=torch.int16).view(torch.bfloat16)
    timing = []
    path = str(tmp_path / "ckpt.bin")
    spill.write_after_dma(path, slot, src, None, 4096, 5.0, timing)
    spill.flush()
    assert timing == [("interval_ns", 10, 20, 4096)]
    assert slot.idle()
    back = torch.zeros(storage.align_up(4096), dtype=torch.uint8)
    spill._file(path).read(back, 0, storage.align_up(4096)).wait()
    assert torch.equal(back[:4096], src.view(torch.uint8))
    spill.close()


def test_stuck_sdma_copy_keeps_its_bounce_slot(monkeypatch, tmp_path):
    """A copy not seen complete within the limit: the write fails with the
    copy's error, and the slot is never handed out again (an engine may still
    write into it)."""
    spill, slot = _spill_with_fake_dma(monkeypatch, tmp_path, stuck=True)
    src = torch.zeros(2048, dtype=torch.bfloat16)
    spill.write_after_dma(str(tmp_path / "ckpt.bin"), slot, src, None, 4096, 5.0)
    with pytest.raises(kernels_mod().DmaCopiesOutstanding):
        spill.flush()
    assert not slot.idle()
    spill._writes.clear()
    spill.close()
