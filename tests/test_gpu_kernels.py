"""HIP kernels through the C ABI, bit-exact against the oracle."""

import os

import numpy as np
import pytest
import torch

import oracle
from conftest import GOLDEN
from test1_amd import kernels
from test1_amd.pinned import pinned_empty

pytestmark = pytest.mark.gpu


def bits16(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().view(torch.int16).numpy().view(np.uint16)


def rand_f32(n, seed, std=0.02):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(n, generator=g) * std


@pytest.mark.parametrize("n", [0, 1, 7, 8, 9, 8191, 8192, 8193, 65536 * 4 + 3, (1 << 20) | 13])
def test_cast_flat_matches_oracle(dev, n):
    x = rand_f32(n, n)
    out = torch.full((n,), 7.0, dtype=torch.bfloat16, device=dev)
    kernels.cast_f32_bf16_(out, x.to(dev))
    torch.cuda.synchronize()
    assert np.array_equal(bits16(out), oracle.cast_f32_bf16(x.numpy()))


@pytest.mark.parametrize("n", [0, 1, 9, 8193, (1 << 20) | 13])
def test_cast_f16_matches_oracle(dev, n):
    """The fp32 -> fp16 staging cast of float16 units: random bit patterns (NaN
    payloads, infinities, subnormals and overflow included) and normal values
    of every magnitude, bit-exact against the oracle (pinned to torch's CPU
    cast); an unaligned view takes the scalar kernel."""
    bits = np.random.default_rng(n).integers(0, 1 << 32, n, dtype=np.uint64).astype(np.uint32)
    x = torch.from_numpy(bits.view(np.float32).copy())
    x[: n // 2] = rand_f32(n // 2, n, std=300.0)
    out = torch.full((n + 1,), 7.0, dtype=torch.float16, device=dev)
    kernels.cast_f32_16_(out[:n], x.to(dev))
    kernels.cast_f32_16_(out[1:n + 1] if n else out[:0], x.to(dev))       # dst off by 2 bytes
    torch.cuda.synchronize()
    exp = oracle.cast_f32_f16(x.numpy())
    assert np.array_equal(bits16(out[1:n + 1]), exp)


def test_cast_golden_and_random_bit_patterns(dev):
    d = np.load(os.path.join(GOLDEN, "cast_f32_bf16.npz"))
    rng = np.random.default_rng(0)
    rnd = rng.integers(0, 1 << 32, 200_003, dtype=np.uint64).astype(np.uint32)  # NaN, inf, denormals included
    bits = np.concatenate([d["x_bits"], rnd])
    x = torch.from_numpy(bits.view(np.float32).copy())
    out = torch.empty(x.numel(), dtype=torch.bfloat16, device=dev)
    kernels.cast_f32_bf16_(out, x.to(dev))
    torch.cuda.synchronize()
    got = bits16(out)
    assert np.array_equal(got[: d["bf16_bits"].size], d["bf16_bits"])
    assert np.array_equal(got, oracle.cast_f32_bf16(bits.view(np.float32)))


@pytest.mark.parametrize("src_off,dst_off", [(1, 0), (0, 3), (5, 5), (2, 6)])
def test_cast_unaligned_views(dev, src_off, dst_off):
    n = 10_007
    x = rand_f32(n + 16, 5)
    xs = x.to(dev)
    out = torch.zeros(n + 16, dtype=torch.bfloat16, device=dev)
    kernels.cast_f32_bf16_(out[dst_off:dst_off + n], xs[src_off:src_off + n])
    torch.cuda.synchronize()
    exp = np.zeros(n + 16, np.uint16)
    exp[dst_off:dst_off + n] = oracle.cast_f32_bf16(x.numpy()[src_off:src_off + n])
    assert np.array_equal(bits16(out), exp)


def test_timed_cast_of_nothing_records_its_events(dev):
    """An empty timed cast launches nothing but still records both events,
    so their elapsed time can be read (and is tiny)."""
    timer = kernels.KernelTimer()
    kernels.cast_f32_bf16_(torch.empty(0, dtype=torch.bfloat16, device=dev), torch.empty(0, device=dev),
                           timer=timer)
    torch.cuda.synchronize()
    assert 0.0 <= timer.elapsed_ms() < 1.0


@pytest.mark.parametrize("n,src_off", [(1 << 20, 0), ((1 << 20) + 5, 0), (4099, 1), (7, 0)])
def test_timed_cast_times_the_kernel_alone(dev, n, src_off):
    """The timed cast (vector kernel, vector + tail, scalar only) gives the
    oracle's bits, and its events time the kernels alone: on a stream that
    first waits for a long matmul on another stream, events recorded around
    the launch include the wait, the kernel-stamped events do not."""
    x = rand_f32(n + src_off, 17)
    xs = x.to(dev)[src_off:]
    out = torch.empty(n, dtype=torch.bfloat16, device=dev)
    a = torch.randn(4096, 4096, device=dev)
    busy, st = torch.cuda.Stream(device=dev), torch.cuda.Stream(device=dev)
    torch.cuda.synchronize()
    with torch.cuda.stream(busy):
        for _ in range(8):
            a = (a @ a).clamp_(-1, 1)
        long_done = torch.cuda.Event()
        long_done.record(busy)
    outer0, outer1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    timer = kernels.KernelTimer()
    outer0.record(st)
    st.wait_event(long_done)
    kernels.cast_f32_bf16_(out, xs, st, timer=timer)
    outer1.record(st)
    torch.cuda.synchronize()
    assert np.array_equal(bits16(out), oracle.cast_f32_bf16(x.numpy()[src_off:]))
    kernel_ms, outer_ms = timer.elapsed_ms(), outer0.elapsed_time(outer1)
    print(f"n={n}: kernel {kernel_ms:.4f} ms, around the wait {outer_ms:.4f} ms")
    assert 0.0 < kernel_ms < 0.5 * outer_ms


def test_cast_full_llama_layer(dev):
    # one Llama-3-8B decoder layer: 218,112,000 elements, the staged unit size
    n = 218_112_000
    x = rand_f32(n, 42)
    out = torch.empty(n, dtype=torch.bfloat16, device=dev)
    kernels.cast_f32_bf16_(out, x.to(dev))
    torch.cuda.synchronize()
    assert np.array_equal(bits16(out), oracle.cast_f32_bf16(x.numpy()))


@pytest.mark.parametrize("n,ws", [(0, 8), (1, 8), (13, 8), (100_003, 4099), ((1 << 22) + 5, 1 << 20),
                                  (1 << 20, 1 << 22)])
def test_stage_pinned_master_through_workspace(dev, n, ws):
    """Pinned fp32 host array -> bf16 device array through a device workspace
    (pieces of the workspace's size rounded down to 8: several pieces, a
    ragged last one, a workspace larger than the array), bit-exact against
    the oracle; the stream's order makes one workspace enough, and the array
    ends where it should (the element after it untouched)."""
    x = pinned_empty(n, torch.float32)
    x.copy_(rand_f32(n, n + 1))
    if n:
        x[0] = float("nan")
    out = torch.full((n + 1,), 7.0, dtype=torch.bfloat16, device=dev)
    work = torch.empty(ws, dtype=torch.float32, device=dev)
    kernels.stage_f32_bf16_(out[:n], x, work)
    torch.cuda.synchronize()
    assert np.array_equal(bits16(out[:n]), oracle.cast_f32_bf16(x.numpy()))
    assert bits16(out[n:])[0] == bits16(torch.tensor([7.0], dtype=torch.bfloat16))[0]


def test_stage_refuses_pageable_host_memory(dev):
    """A pageable source cannot be copied asynchronously: the library says so
    before it enqueues anything (checked in C, below the Python wrapper)."""
    from test1_amd import _native

    x = torch.randn(1000)                      # pageable
    out = torch.empty(1000, dtype=torch.bfloat16, device=dev)
    work = torch.empty(256, dtype=torch.float32, device=dev)
    with pytest.raises(ValueError, match="pinned"):
        kernels.stage_f32_bf16_(out, x, work)
    rc = _native.hip().sf_stage_f32_bf16(x.data_ptr(), out.data_ptr(), 1000, work.data_ptr(), 256, None)
    assert rc == _native.SF_EINVAL


def test_cast_scatter_segments(dev):
    # 70 segments (> one launch's 64), ragged sizes, some misaligned, one empty
    rng = np.random.default_rng(1)
    sizes = [int(s) for s in rng.integers(0, 20_000, 70)]
    sizes[3] = 0
    src = rand_f32(sum(sizes) + 3 * 70, 9).to(dev)
    dst = torch.zeros(sum(sizes) + 8 * 70, dtype=torch.bfloat16, device=dev)
    pairs, so, do, expect = [], 0, 0, np.zeros(dst.numel(), np.uint16)
    host = src.cpu().numpy()
    for k, n in enumerate(sizes):
        so += k % 3          # skew the source alignment
        do += (k * 5) % 8    # and the destination alignment
        pairs.append((src[so:so + n], dst[do:do + n]))
        expect[do:do + n] = oracle.cast_f32_bf16(host[so:so + n])
        so += n
        do += n
    kernels.cast_scatter_f32_bf16(pairs)
    torch.cuda.synchronize()
    assert np.array_equal(bits16(dst), expect)


def test_pack_unpack_round_trip(dev):
    g = torch.Generator().manual_seed(3)
    sizes = [16_777_216 // 64, 4096, 4096 + 3, 1, 0, 8192 * 4 + 9]
    parts = [torch.randn(n, generator=g).bfloat16() for n in sizes]
    dparts = [p.to(dev) for p in parts]
    packed = torch.empty(sum(sizes) + 5, dtype=torch.bfloat16, device=dev)
    kernels.pack_b16(dparts, packed)
    torch.cuda.synchronize()
    exp = oracle.pack_b16([p.view(torch.int16).numpy() for p in parts])
    assert np.array_equal(bits16(packed)[: exp.size], exp)
    outs = [torch.zeros_like(p) for p in dparts]
    kernels.unpack_b16(packed, outs)
    torch.cuda.synchronize()
    for a, b in zip(outs, parts):
        assert torch.equal(a.cpu().view(torch.int16), b.view(torch.int16))


def test_copy_segs_and_fill(dev):
    a = torch.arange(50_000, dtype=torch.int16, device=dev)
    b = torch.zeros(60_000, dtype=torch.int16, device=dev)
    kernels.copy_segs_b16([(a[1:10_001], b[3:10_003]), (a[20_000:20_008], b[40_000:40_008])])
    kernels.fill_b16_(b[50_001:59_999], 0x1234)
    torch.cuda.synchronize()
    exp = np.zeros(60_000, np.int16)
    exp[3:10_003] = np.arange(1, 10_001)
    exp[40_000:40_008] = np.arange(20_000, 20_008)
    exp[50_001:59_999] = 0x1234
    assert np.array_equal(b.cpu().numpy(), exp)


def test_fill_and_cast_in_a_captured_graph(dev):
    """``sf_fill_b16`` and ``sf_cast_f32_bf16`` are plain kernel launches, so
    they can be captured in a HIP graph: four replays, each after eager work
    that overwrites both outputs and a synchronisation, give the fill pattern
    and the oracle's cast every time."""
    n = (1 << 20) + 13
    src = rand_f32(n, seed=11).to(dev)
    dst = torch.zeros(n, dtype=torch.bfloat16, device=dev)
    buf = torch.zeros(70_000, dtype=torch.int16, device=dev)
    expect_cast = oracle.cast_f32_bf16(src.cpu().numpy())
    expect_fill = np.zeros(70_000, np.int16)
    expect_fill[3:69_998] = 0x1234
    # warm up on a side stream (the kernels' first launches load their code)
    side = torch.cuda.Stream(device=dev)
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        kernels.fill_b16_(buf[3:69_998], 0x1234)
        kernels.cast_f32_bf16_(dst, src)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        kernels.fill_b16_(buf[3:69_998], 0x1234)
        kernels.cast_f32_bf16_(dst, src)
    for rep in range(4):
        buf.fill_(-(rep + 1))
        buf[:3] = 0
        buf[69_998:] = 0
        dst.fill_(float(rep + 7))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(buf.cpu().numpy(), expect_fill), rep
        assert np.array_equal(bits16(dst), expect_cast), rep


def test_pinned_memcpy_round_trip(dev):
    n = 3 * (1 << 20) + 7
    h = pinned_empty(n, torch.float32)
    assert h.is_pinned()
    h.copy_(rand_f32(n, 11))
    d = torch.empty(n, dtype=torch.float32, device=dev)
    back = pinned_empty(n, torch.float32)
    s = torch.cuda.Stream()
    kernels.memcpy_async(d, h, s)
    kernels.memcpy_async(back, d, s)
    s.synchronize()
    assert torch.equal(back.view(torch.int32), h.view(torch.int32))


@pytest.mark.parametrize("max_wg", [1, 8, 64, 0])
def test_pack_into_pinned_host_memory(dev, max_wg):
    """The grad offload path: one kernel gathers device tensors straight into a
    pinned host slot, with a capped grid that strides over all tiles."""
    g = torch.Generator().manual_seed(21)
    sizes = [8192 * 7 + 3, 5, 0, 4096 * 33, 1]
    parts = [torch.randn(n, generator=g).bfloat16() for n in sizes]
    host = pinned_empty(sum(sizes) + 11, torch.bfloat16)
    host.view(torch.int16).fill_(-1)
    s = torch.cuda.Stream()
    kernels.pack_b16([p.to(dev) for p in parts], host, s, max_workgroups=max_wg)
    s.synchronize()
    exp = oracle.pack_b16([p.view(torch.int16).numpy() for p in parts])
    got = host.view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got[: exp.size], exp)
    assert np.all(got[exp.size:] == 0xFFFF)  # nothing written past the packed range


def test_copy_segs_to_pinned_host_offsets(dev):
    a = torch.arange(100_000, dtype=torch.int16, device=dev)
    host = pinned_empty(120_000, torch.int16)
    host.zero_()
    kernels.copy_segs_b16([(a[:70_001], host[7:70_008]), (a[90_000:], host[110_000:])], max_workgroups=4)
    torch.cuda.synchronize()
    exp = np.zeros(120_000, np.int16)
    exp[7:70_008] = np.arange(70_001)
    exp[110_000:] = np.arange(90_000, 100_000)
    assert np.array_equal(host.numpy(), exp)


def test_sdma_copy_d2h(dev):
    """Device -> pinned host over an SDMA engine, several segments, bit-exact."""
    kernels.dma_init(dev)
    g = torch.Generator().manual_seed(5)
    parts = [torch.randn(n, generator=g).bfloat16() for n in (1 << 20, 7, 4096 * 3 + 1)]
    dparts = [p.to(dev) for p in parts]
    host = pinned_empty(sum(p.numel() for p in parts), torch.bfloat16)
    torch.cuda.synchronize()
    pairs, off = [], 0
    for p in dparts:
        pairs.append((p, host[off:off + p.numel()]))
        off += p.numel()
    h = kernels.dma_copy_d2h(pairs)
    kernels.dma_wait(h)
    exp = oracle.pack_b16([p.view(torch.int16).numpy() for p in parts])
    assert np.array_equal(host.view(torch.int16).numpy().view(np.uint16), exp)


def test_sdma_copy_d2h_routes_around_engine_held_by_waiting_hip_copy(dev):
    """A HIP host -> device copy ordered after an event that has not fired
    holds its SDMA engine until the event fires.  With routing on (mode 1)
    and engines 0 and 1 selected (the ones HIP's host -> device copies take
    first), a device -> host copy issued meanwhile must not queue behind such
    copies: it completes while the event is still pending, with exact
    bytes."""
    kernels.dma_init(dev)
    saved = kernels.dma_engines()
    nb = 64 << 20
    hsrc = pinned_empty(nb, torch.uint8)
    dbufs = [torch.empty(nb, dtype=torch.uint8, device=dev) for _ in range(2)]
    src = torch.randint(0, 256, (nb // 4,), dtype=torch.int32, device=dev).view(torch.uint8)
    host = pinned_empty(nb, torch.uint8)
    host.zero_()
    spin, sa, sc = torch.cuda.Stream(dev), torch.cuda.Stream(dev), torch.cuda.Stream(dev)
    # spin length for about 0.3 s, from a short timed spin
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(spin):
        t0.record()
        torch.cuda._sleep(5_000_000)
        t1.record()
    t1.synchronize()
    cycles = int(min(5_000_000 * 300.0 / max(t0.elapsed_time(t1), 1e-3), 2_000_000_000))
    for s in (sa, sc):  # first copies on these streams, outside the test window
        kernels.memcpy_async(dbufs[0], hsrc, s)
    torch.cuda.synchronize()
    with torch.cuda.stream(spin):
        torch.cuda._sleep(cycles)
    ev = torch.cuda.Event()
    ev.record(spin)
    for s, d in zip((sa, sc), dbufs):
        s.wait_event(ev)
        kernels.memcpy_async(d, hsrc, s)
    try:
        kernels.dma_set_engines([0, 1])
        kernels.dma_set_avoid_held(1)
        h = kernels.dma_copy_d2h([(src, host)])
        kernels.dma_wait(h)
        pending_after_copy = not ev.query()
    finally:
        kernels.dma_set_avoid_held(0)
        kernels.dma_set_engines(saved)
        torch.cuda.synchronize()
    assert pending_after_copy, "the device -> host copy waited for the held engines"
    assert torch.equal(host, src.cpu())


def test_sdma_copy_d2h_default_engine_clear_of_waiting_hip_copies(dev):
    """HIP puts a host -> device copy on the first free SDMA engine (0, then
    1, then 2), and a copy ordered after an event that has not fired holds
    its engine until the event fires.  With three such copies pending (on
    engines 0, 1 and 2), a device -> host copy on the library's default
    engine completes while the event is still pending, with exact bytes."""
    kernels.dma_init(dev)
    if os.environ.get("SF_DMA_ENGINES"):
        pytest.skip("SF_DMA_ENGINES overrides the default engine")
    assert kernels.dma_engines() == [3]
    nb = 64 << 20
    hsrc = pinned_empty(nb, torch.uint8)
    dbufs = [torch.empty(nb, dtype=torch.uint8, device=dev) for _ in range(3)]
    src = torch.randint(0, 256, (nb // 4,), dtype=torch.int32, device=dev).view(torch.uint8)
    host = pinned_empty(nb, torch.uint8)
    host.zero_()
    spin = torch.cuda.Stream(dev)
    streams = [torch.cuda.Stream(dev) for _ in range(3)]
    # spin length for about 0.3 s, from a short timed spin
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(spin):
        t0.record()
        torch.cuda._sleep(5_000_000)
        t1.record()
    t1.synchronize()
    cycles = int(min(5_000_000 * 300.0 / max(t0.elapsed_time(t1), 1e-3), 2_000_000_000))
    for s in streams:  # first copies on these streams, outside the test window
        kernels.memcpy_async(dbufs[0], hsrc, s)
    torch.cuda.synchronize()
    with torch.cuda.stream(spin):
        torch.cuda._sleep(cycles)
    ev = torch.cuda.Event()
    ev.record(spin)
    for s, d in zip(streams, dbufs):
        s.wait_event(ev)
        kernels.memcpy_async(d, hsrc, s)
    try:
        h = kernels.dma_copy_d2h([(src, host)])
        kernels.dma_wait(h)
        pending_after_copy = not ev.query()
    finally:
        torch.cuda.synchronize()
    assert pending_after_copy, "the device -> host copy waited behind HIP copies held by a pending event"
    assert torch.equal(host, src.cpu())


@pytest.mark.parametrize("row_len", [4096, 5120, 8192, 8200, 24, 13])
def test_gather_rows_from_pinned_host_table(dev, row_len):
    # fp32 rows read by the kernel from pinned host memory, rounded to bf16:
    # equal to the oracle cast of the same rows (vector path for row_len % 8
    # == 0, scalar path otherwise), repeated ids included.  Row lengths cover
    # 2 and 2.5 groups of 8 per lane, exactly one pass of 4 groups per lane
    # (8192) and a second pass with one group for the first lane (8200).
    V, ntok = 257, 300
    table = pinned_empty((V, row_len), torch.float32)
    table.copy_(rand_f32(V * row_len, row_len).view(V, row_len))
    ids = torch.from_numpy(np.random.default_rng(row_len).integers(0, V, ntok)).to(dev)
    out = torch.full((ntok, row_len), 3.0, dtype=torch.bfloat16, device=dev)
    bad = torch.zeros(1, dtype=torch.int32, device=dev)
    kernels.gather_rows(table, ids, out, bad=bad)
    torch.cuda.synchronize()
    exp = oracle.cast_f32_bf16(table.numpy()[ids.cpu().numpy()].reshape(-1))
    assert np.array_equal(bits16(out).reshape(-1), exp)
    assert int(bad.item()) == 0


@pytest.mark.parametrize("H", [128, 5120, 8200])
def test_gather_rows_b16_into_pinned_host_and_bad_ids(dev, H):
    # 16-bit rows copied from device memory into pinned host memory by a
    # capped grid (the gradient-row offload); ids out of range give 0xFFFF
    # rows and raise the flag, in-range rows are unaffected.
    V = 64
    table = torch.randn(V, H, device=dev).bfloat16()
    ids = torch.tensor([3, 0, 63, 64, -1, 3, 17], dtype=torch.int64, device=dev)
    out = pinned_empty((ids.numel(), H), torch.bfloat16)
    bad = pinned_empty(1, torch.int32)
    bad.zero_()
    kernels.gather_rows(table, ids, out, bad=bad, max_workgroups=2)
    torch.cuda.synchronize()
    t = bits16(table)
    o = bits16(out)
    for k, r in enumerate(ids.tolist()):
        if 0 <= r < V:
            assert np.array_equal(o[k], t[r]), k
        else:
            assert (o[k] == 0xFFFF).all(), k
    assert int(bad[0]) == 1
