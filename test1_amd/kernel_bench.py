"""Microbenchmark of the staging kernels at one unit's size.

    python -m test1_amd.kernel_bench [--elements N] [--reps R]

Times, with HIP events on the stream each runs on:
  cast      sf_cast_f32_bf16 over N fp32 elements (6 B per element of HBM)
  copy      a plain device copy of N/2 fp32 elements (8 B per element),
            the reference point for hardware counters (FETCH_SIZE and
            WRITE_SIZE are scaled by what they read for it)
  pack_d2h  sf_pack_b16 of N/2 bf16 elements into pinned host memory with
            the offload path's 16-workgroup grid (host link)
  h2d       one DMA copy of N fp32 elements from pinned host memory
Default N is one Llama-3-8B decoder layer (218,112,000 parameters).

With ``--rotate K`` the cast cycles through K source/destination pairs, so
that a launch does not find its input in the 256 MB Infinity Cache left by
the previous one (pick K with K * 6 * N well above that size for small N).

With ``--gap-ms G`` the cast is also timed alone after G ms with the GPU
idle before each launch (a host sleep after a synchronisation), as a unit's
cast runs in a step whose compute stream waited for the unit's copy: each
launch timed by the events the runtime stamps around the kernel itself.

With ``--beside-h2d-streams K`` the cast on the default stream is timed
beside a layer's host-to-device copy issued on each of K new streams in turn,
with and without an event recorded behind the copy (the hardware queue a
stream gets at its first use decides whether such a copy slows the cast).
"""

from __future__ import annotations

import argparse
import json

import torch

from . import kernels
from .pinned import pinned_empty

HBM_PEAK_GBS = 8000.0


def _time(fn, stream, reps):
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(reps):
        fn()
    e1.record(stream)
    e1.synchronize()
    return e0.elapsed_time(e1) / reps


def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("--elements", type=int, default=218_112_000)
    ap.add_argument("--reps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--rotate", type=int, default=1, help="source/destination pairs the cast cycles through")
    ap.add_argument("--gap-ms", type=float, default=0.0,
                    help="also time the cast after this many ms of idle GPU before each launch")
    ap.add_argument("--beside-h2d", action="store_true",
                    help="also time the cast while a host-to-device copy runs on another stream")
    ap.add_argument("--after-h2d", action="store_true",
                    help="also time the cast right after a host-to-device copy wrote its source (same stream)")
    ap.add_argument("--streamed", action="store_true",
                    help="also time casts that each wait (cross-stream event) for the copy of their source, with "
                         "the copies queued back to back on another stream, as in the pool schedule's forward")
    ap.add_argument("--beside-sdma-d2h", action="store_true",
                    help="also time the cast while device-to-host copies run on the gradient SDMA engines")
    ap.add_argument("--beside-h2d-streams", type=int, default=0, metavar="K",
                    help="also time the cast on the default stream beside a host-to-device copy with an event "
                         "recorded behind it, from each of K new streams first used in turn (the HIP runtime "
                         "gives a stream its hardware queue at first use), and without the event")
    args = ap.parse_args(argv)
    n, reps = args.elements, args.reps
    dev = torch.device("cuda", 0)
    s = torch.cuda.current_stream()
    pairs = [(torch.randn(n, device=dev) * 0.02, torch.empty(n, dtype=torch.bfloat16, device=dev))
             for _ in range(max(1, args.rotate))]
    src, dst = pairs[0]
    half = n // 2
    cp_src = torch.ones(half, dtype=torch.float32, device=dev)
    cp_dst = torch.empty_like(cp_src)
    g = torch.ones(half, dtype=torch.bfloat16, device=dev)
    host_g = pinned_empty(half, torch.bfloat16)
    host_w = pinned_empty(n, torch.float32)
    host_w.fill_(0.5)
    dev_w = torch.empty(n, dtype=torch.float32, device=dev)
    for _ in range(args.warmup):
        kernels.cast_f32_bf16_(dst, src, s)
        cp_dst.copy_(cp_src)
    torch.cuda.synchronize()
    res = {}
    nxt = iter(range(1 << 62))

    def cast_next():
        a, b = pairs[next(nxt) % len(pairs)]
        kernels.cast_f32_bf16_(b, a, s)

    ms = _time(cast_next, s, reps)
    res["cast"] = {"ms": ms, "GB/s": 6 * n / ms / 1e6, "frac_hbm": 6 * n / ms / 1e6 / HBM_PEAK_GBS,
                   "algorithmic_bytes": 6 * n, "rotated_pairs": len(pairs)}
    if args.gap_ms > 0:
        import time

        timers = []
        for k in range(reps):
            torch.cuda.synchronize()
            time.sleep(args.gap_ms * 1e-3)
            t = kernels.KernelTimer()
            a, b = pairs[k % len(pairs)]
            kernels.cast_f32_bf16_(b, a, s, timer=t)
            timers.append(t)
        torch.cuda.synchronize()
        each = [t.elapsed_ms() for t in timers]
        ms = sum(each) / len(each)
        res["cast_after_idle"] = {"gap_ms": args.gap_ms, "ms": ms, "min_ms": min(each), "max_ms": max(each),
                                  "GB/s": 6 * n / ms / 1e6, "frac_hbm": 6 * n / ms / 1e6 / HBM_PEAK_GBS}
        timers = []
        for k in range(reps):
            t = kernels.KernelTimer()
            a, b = pairs[k % len(pairs)]
            kernels.cast_f32_bf16_(b, a, s, timer=t)
            timers.append(t)
        torch.cuda.synchronize()
        ms = sum(t.elapsed_ms() for t in timers) / reps
        res["cast_back_to_back"] = {"ms": ms, "GB/s": 6 * n / ms / 1e6, "frac_hbm": 6 * n / ms / 1e6 / HBM_PEAK_GBS}
    if args.beside_h2d:
        other = torch.cuda.Stream(device=dev)
        dev_w2 = torch.empty(n, dtype=torch.float32, device=dev)
        torch.cuda.synchronize()
        with torch.cuda.stream(other):
            for _ in range(4):       # ~65 ms of copying, longer than the casts below
                dev_w2.copy_(host_w, non_blocking=True)
        timers = []
        for k in range(reps):
            t = kernels.KernelTimer()
            a, b = pairs[k % len(pairs)]
            kernels.cast_f32_bf16_(b, a, s, timer=t)
            timers.append(t)
        torch.cuda.synchronize()
        ms = sum(t.elapsed_ms() for t in timers) / reps
        res["cast_beside_h2d"] = {"ms": ms, "GB/s": 6 * n / ms / 1e6, "frac_hbm": 6 * n / ms / 1e6 / HBM_PEAK_GBS}
        del dev_w2
    if args.after_h2d:
        timers = []
        for k in range(reps):
            a, b = pairs[k % len(pairs)]
            kernels.memcpy_async(a, host_w, s)      # the source freshly written by DMA
            t = kernels.KernelTimer()
            kernels.cast_f32_bf16_(b, a, s, timer=t)
            timers.append(t)
        torch.cuda.synchronize()
        ms = sum(t.elapsed_ms() for t in timers) / reps
        res["cast_after_h2d_of_its_source"] = {"ms": ms, "GB/s": 6 * n / ms / 1e6,
                                               "frac_hbm": 6 * n / ms / 1e6 / HBM_PEAK_GBS}
        # the same launches with the copy into the other pair's source: the
        # cast reads data written long before
        timers = []
        for k in range(reps):
            a, b = pairs[k % len(pairs)]
            c, _ = pairs[(k + 1) % len(pairs)]
            kernels.memcpy_async(c, host_w, s)
            t = kernels.KernelTimer()
            kernels.cast_f32_bf16_(b, a, s, timer=t)
            timers.append(t)
        torch.cuda.synchronize()
        ms = sum(t.elapsed_ms() for t in timers) / reps
        res["cast_after_h2d_of_another_buffer"] = {"ms": ms, "GB/s": 6 * n / ms / 1e6,
                                                   "frac_hbm": 6 * n / ms / 1e6 / HBM_PEAK_GBS}
    if args.streamed:
        up = torch.cuda.Stream(device=dev)
        torch.cuda.synchronize()
        evs = []
        for k in range(reps):
            a, _ = pairs[k % len(pairs)]
            if k >= len(pairs):
                up.wait_event(evs[k - len(pairs)][1])   # the source's previous cast has read it
            kernels.memcpy_async(a, host_w, up)
            ev = torch.cuda.Event()
            ev.record(up)
            t = kernels.KernelTimer()
            s.wait_event(ev)
            kernels.cast_f32_bf16_(pairs[k % len(pairs)][1], a, s, timer=t)
            done = torch.cuda.Event()
            done.record(s)
            evs.append((t, done))
        torch.cuda.synchronize()
        each = [t.elapsed_ms() for t, _ in evs]
        ms = sum(each) / len(each)
        res["cast_streamed"] = {"ms": ms, "min_ms": min(each), "max_ms": max(each), "GB/s": 6 * n / ms / 1e6,
                                "frac_hbm": 6 * n / ms / 1e6 / HBM_PEAK_GBS}
    if args.beside_sdma_d2h:
        kernels.dma_init(dev)
        host_big = pinned_empty(4 * n, torch.bfloat16)
        src_big = torch.ones(n, dtype=torch.bfloat16, device=dev)
        torch.cuda.synchronize()
        # ~4 x 436 MB at ~50 GB/s: longer than the casts below
        handle = kernels.dma_copy_d2h([(src_big, host_big[k * n:(k + 1) * n]) for k in range(4)])
        timers = []
        for k in range(reps):
            t = kernels.KernelTimer()
            a, b = pairs[k % len(pairs)]
            kernels.cast_f32_bf16_(b, a, s, timer=t)
            timers.append(t)
        torch.cuda.synchronize()
        busy = not kernels.dma_query(handle)
        kernels.DmaReady(handle, timeout=60).release()
        ms = sum(t.elapsed_ms() for t in timers) / reps
        res["cast_beside_sdma_d2h"] = {"ms": ms, "GB/s": 6 * n / ms / 1e6, "frac_hbm": 6 * n / ms / 1e6 / HBM_PEAK_GBS,
                                       "copies_still_running_after_the_casts": busy}
        del host_big, src_big
    if args.beside_h2d_streams > 0:
        streams = []
        for _ in range(args.beside_h2d_streams):
            st = torch.cuda.Stream(device=dev)
            torch.cuda.Event().record(st)         # first use: the stream's hardware queue
            streams.append(st)
        torch.cuda.synchronize()
        nc = min(reps, 8)                          # ~2 ms of casts, inside one ~17 ms copy of a layer

        def beside(st, with_event):
            torch.cuda.synchronize()
            kernels.memcpy_async(dev_w, host_w, st)
            if with_event:
                torch.cuda.Event().record(st)
            timers = []
            for k in range(nc):
                t = kernels.KernelTimer()
                a, b = pairs[k % len(pairs)]
                kernels.cast_f32_bf16_(b, a, s, timer=t)
                timers.append(t)
            torch.cuda.synchronize()
            ms = sum(t.elapsed_ms() for t in timers) / nc
            return round(6 * n / ms / 1e6 / HBM_PEAK_GBS, 4)

        res["cast_beside_h2d_streams"] = {
            "frac_hbm_with_event": [beside(st, True) for st in streams],
            "frac_hbm_without_event": [beside(st, False) for st in streams],
            "streams_in_first_use_order": len(streams)}
    ms = _time(lambda: cp_dst.copy_(cp_src), s, reps)
    res["copy"] = {"ms": ms, "GB/s": 8 * half / ms / 1e6, "bytes_read": 4 * half, "bytes_written": 4 * half}
    ms = _time(lambda: kernels.pack_b16([g], host_g, s, max_workgroups=16), s, max(1, reps // 4))
    res["pack_d2h"] = {"ms": ms, "GB/s": 2 * half / ms / 1e6}
    ms = _time(lambda: kernels.memcpy_async(dev_w, host_w, s), s, max(1, reps // 4))
    res["h2d"] = {"ms": ms, "GB/s": 4 * n / ms / 1e6}
    print(json.dumps({"elements": n, "reps": reps, **res}), flush=True)


if __name__ == "__main__":
    main()
