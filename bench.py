#!/usr/bin/env python3
"""Benchmark of the single-GPU layer-streaming training step.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME]

Default workload ``llama3-8b``: one causal-LM training step of a Llama-3.1-8B
shaped model (32 layers, hidden 4096, 32/8 heads of 128, intermediate 14336,
vocab 128256, RoPE theta 500000), random N(0, 0.02) weights, batch 4 x 1024
uniform random tokens, through SlideFSDP: fp32 masters in pinned host
memory, layer-wise H2D + on-GPU cast, checkpointed activations offloaded to
host, bf16 grads D2H into the host LayerAdam.  Other workloads:
``qwen2.5-14b`` (48 layers, hidden 5120, batch 2 x 4096), ``tiny`` (a small
Llama for a quick check).

One JSON line is printed with the metric (tokens/s), the roofline of the
staging cast kernel (HBM-bound, measured with HIP events on its stream over
the timed region), the host-link-bound kernels beside it (checkpoint pack,
embedding row gathers), the host link per direction (rate over the union of
all transfers' intervals, the fraction of that time under layer compute, and
plain pinned copies for the rate this box reaches), and the reference's
host-side staging + AdamW path restated with this build's code and timed on
this machine's cores (``cpu_baseline``).  ``variants`` holds shorter timed
runs on the same model: ``pool``, the reference's schedule (every unit in the
2-unit pool and reloaded for its backward), and the other parameter H2D
format (fp32 masters + GPU cast, or the host optimizer's bf16 copy).
"""

from __future__ import annotations

import argparse
import itertools
import json
import math
import os
import sys
import time
from concurrent.futures import ThreadPoolExecutor
from typing import Optional

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0     # MI355X HBM3E, GB/s
LINK_PEAK_GBS = 63.0      # PCIe 5.0 x16, per direction, GB/s
D2H_WORKGROUPS = 16       # grid of the kernels writing into pinned host memory (the runtime's default)

WORKLOADS = {
    "llama3-8b": dict(vocab=128256, hidden=4096, inter=14336, layers=32, heads=32, kv=8, head_dim=128,
                      theta=500000.0, batch=4, seq=1024, model="Llama-3.1-8B", arch="llama"),
    "qwen2.5-14b": dict(vocab=152064, hidden=5120, inter=13824, layers=48, heads=40, kv=8, head_dim=128,
                        theta=1000000.0, batch=2, seq=4096, model="Qwen2.5-14B", arch="qwen2"),
    "tiny": dict(vocab=4096, hidden=512, inter=1024, layers=4, heads=8, kv=4, head_dim=64,
                 theta=500000.0, batch=2, seq=256, model="tiny-llama", arch="llama"),
}


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def build_model(w: dict, seed: int = 42):
    """Random-init model of the workload's architecture, N(0, 0.02) weights and
    unit RMSNorm weights, built without materialising HF's own init."""
    import torch

    if w["arch"] == "llama":
        from transformers import LlamaConfig as C, LlamaForCausalLM as M
    else:
        from transformers import Qwen2Config as C, Qwen2ForCausalLM as M
    cfg = C(vocab_size=w["vocab"], hidden_size=w["hidden"], intermediate_size=w["inter"],
            num_hidden_layers=w["layers"], num_attention_heads=w["heads"], num_key_value_heads=w["kv"],
            head_dim=w["head_dim"], rope_theta=w["theta"], max_position_embeddings=max(8192, w["seq"]),
            tie_word_embeddings=False, torch_dtype=torch.float32)
    cfg._attn_implementation = "sdpa"
    with torch.device("meta"):
        model = M(cfg)
    model = model.to_empty(device="cpu")
    # buffers created on meta (rotary inv_freq) must be rebuilt on the host
    rope_cls = type(model.model.rotary_emb)
    model.model.rotary_emb = rope_cls(config=cfg)
    params = list(model.named_parameters())

    def init(i_np):
        i, (name, p) = i_np
        g = torch.Generator().manual_seed(seed * 100003 + i)
        with torch.no_grad():
            if "norm" in name:
                p.fill_(1.0)
            elif name.endswith(".bias"):
                p.zero_()
            else:
                p.normal_(0.0, 0.02, generator=g)

    with ThreadPoolExecutor(max_workers=min(16, os.cpu_count() or 1)) as ex:
        list(ex.map(init, enumerate(params)))
    return model


def traffic_factor():
    """HBM bytes moved per algorithmic byte of the staging cast, from the
    FETCH_SIZE / WRITE_SIZE counter runs summarised under profiles/ (None if
    that summary is absent)."""
    import re

    path = os.path.join(ROOT, "profiles", "cast_flat_kernel__pmc_llama3_8b_layer.md")
    try:
        m = re.search(r"traffic_per_algorithmic_byte:\s*([0-9.]+)", open(path).read())
    except OSError:
        return None
    return float(m.group(1)) if m else None


def _untimed(rec) -> bool:
    """("untimed", bytes): SDMA copies whose engine timestamps were not
    available (a profiler tracing async copies takes them over)."""
    return isinstance(rec[0], str) and rec[0] == "untimed"


def elapsed_stats(records):
    """(busy ms, total bytes or elements) from (start_event, end_event, amount)
    or (KernelTimer, None, amount) records (summed) or ("interval_ns", start,
    end, amount) records of copies
    that may overlap one another (busy = union of the intervals)."""
    ms = amt = 0.0
    intervals = []
    for r in records or []:
        if _untimed(r):
            continue
        if len(r) == 4:
            intervals.append((r[1], r[2]))
            amt += r[3]
        elif r[1] is None:   # a KernelTimer: the kernels' own start and end
            ms += r[0].elapsed_ms()
            amt += r[2]
        else:
            ms += r[0].elapsed_time(r[1])
            amt += r[2]
    intervals.sort()
    cur_s = cur_e = None
    for s, e in intervals:
        if cur_e is None or s > cur_e:
            if cur_e is not None:
                ms += (cur_e - cur_s) * 1e-6
            cur_s, cur_e = s, e
        else:
            cur_e = max(cur_e, e)
    if cur_e is not None:
        ms += (cur_e - cur_s) * 1e-6
    return ms, amt


# One Llama-3-8B decoder layer's parameters in named_parameters() order.
LLAMA3_8B_LAYER_SHAPES = [(4096, 4096), (1024, 4096), (1024, 4096), (4096, 4096), (14336, 4096), (14336, 4096),
                          (4096, 14336), (4096,), (4096,)]


def cpu_baseline(total_params: int, tokens: int, resident_params: int, min_seconds: float = 10.0,
                 warmup: int = 3):
    """The reference's host-side work per unit, timed on this host's cores on
    a sample of one Llama-3-8B decoder layer (218,112,000 parameters, seed
    42), restated with this build's own code: the fp32 -> bf16 cast of the
    flat master (torch CPU ``copy_``, the call of reference layer_state.py:301)
    for each load, ``grad.float()`` per parameter (layer_adam.py:404) and the
    AdamW per parameter through the reference's ``cpu_adam.adam_update``
    interface (layer_adam.py:405-425; this build's AVX-512 implementation,
    bit-exact with the reference's).  Scaled to the model: the per-parameter
    cost times its parameters, the cast counted twice per step (forward and
    backward loads) except for the units that stay loaded.  Timed iterations
    run until ``min_seconds`` of CPU work (at least 5)."""
    import torch

    from test1_amd.optimizer import cpu_adam

    threads = torch.get_num_threads()
    g = torch.Generator().manual_seed(42)
    sizes = [int(torch.Size(s).numel()) for s in LLAMA3_8B_LAYER_SHAPES]
    n = sum(sizes)
    master = torch.randn(n, generator=g) * 0.02
    bf = torch.empty(n, dtype=torch.bfloat16)
    grad = (torch.randn(n, generator=g) * 1e-3).bfloat16()
    m = torch.zeros(n)
    v = torch.zeros(n)
    offs = [sum(sizes[:i]) for i in range(len(sizes))]
    views = [(master[o:o + k], grad[o:o + k], m[o:o + k], v[o:o + k]) for o, k in zip(offs, sizes)]
    opt_id = 77
    cpu_adam.create_adam(opt_id, 1e-5, 0.9, 0.999, 1e-8, 0.01, True, False)
    t_cast = t_unpack = t_adam = 0.0
    t_all = time.perf_counter()
    iters = 0
    t_timed = None
    try:
        for it in itertools.count():
            if it == warmup:
                t_timed = time.perf_counter()
            if t_timed is not None and iters >= 5 and time.perf_counter() - t_timed >= min_seconds:
                break
            t0 = time.perf_counter()
            bf.copy_(master)
            t1 = time.perf_counter()
            dt_unpack = dt_adam = 0.0
            for p, gb, mm, vv in views:
                a = time.perf_counter()
                gf = gb.float()
                b = time.perf_counter()
                cpu_adam.adam_update(opt_id, it + 1, 1e-5, 0.9, 0.999, 1e-8, 0.01, True, p, gf, mm, vv)
                dt_unpack += b - a
                dt_adam += time.perf_counter() - b
            if it >= warmup:
                t_cast += t1 - t0
                t_unpack += dt_unpack
                t_adam += dt_adam
                iters += 1
    finally:
        cpu_adam.destroy_adam(opt_id)
    t_all = time.perf_counter() - t_all
    t_cast, t_unpack, t_adam = (x / iters for x in (t_cast, t_unpack, t_adam))
    per_param = (t_cast * 2 + t_unpack + t_adam) / n
    # units that stay resident are cast once per step, not twice
    step_s = per_param * total_params - t_cast / n * resident_params
    return {
        "value": tokens / step_s,
        "unit": "tokens/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"one Llama-3-8B decoder layer ({n:,} params in its 9 parameters), {warmup} warmup + "
                   f"{iters} timed iterations ({t_all:.1f} s of CPU work) on {threads} threads: torch CPU "
                   f"fp32->bf16 cast {t_cast * 1e3:.1f} ms, grad.float() per parameter {t_unpack * 1e3:.1f} ms, "
                   f"AdamW per parameter (this build's AVX-512 cpu_adam, reference call pattern) "
                   f"{t_adam * 1e3:.1f} ms ({28 * n / t_adam / 1e9:.1f} GB/s at 28 B/param); per-step time = "
                   f"per-parameter cost x {total_params:,} params (cast twice, resident units once)"),
        "ms_per_layer": {"cast": t_cast * 1e3, "unpack": t_unpack * 1e3, "adam": t_adam * 1e3},
        "adam_gbs": 28 * n / t_adam / 1e9,
    }


def timed_run(model, w: dict, args, dev, h2d_format: str, resident_layers, d2h_engine: str,
              timeline: str = "", batch_seed: int = 0, steps: Optional[int] = None,
              warmup: Optional[int] = None, after=None) -> dict:
    """Wrap ``model`` in SlideFSDP, run the warmup steps, then time
    ``args.steps`` steps between two device synchronisations.  Returns the
    timings and the per-kernel / per-copy event records; closes the wrapper.
    A second run on the same model uses another ``batch_seed``: the first
    run's updates lower the loss on the batches it saw.  ``after(sf)``, if
    given, runs once the timed steps are done, before the wrapper closes;
    its result is returned as ``after``."""
    import gc

    import torch

    from test1_amd import SlideFSDP, SlideFSDPConfig

    t0 = time.time()
    cfg = SlideFSDPConfig(device=dev, lr=1e-5, weight_decay=0.01, attention_implementation="sdpa",
                          ac_offload_mode=args.ac_offload, gpu_buffer_pool_size=args.pool_size,
                          ac_offload_dir=os.path.join(args.offload_dir, "activations"),
                          optimizer_nvme_offload_fraction=args.opt_nvme_fraction,
                          optimizer_offload_dir=os.path.join(args.offload_dir, "optimizer"),
                          enable_activation_checkpoint=not args.no_activation_checkpoint)
    kw = {}
    if args.wait_timeout is not None:
        kw["wait_timeout"] = args.wait_timeout if args.wait_timeout > 0 else None
    sf = SlideFSDP(model, cfg, d2h_engine=d2h_engine, h2d_format=h2d_format, resident_layers=resident_layers,
                   fused_cross_entropy=args.fused_ce, update_piece_elems=args.piece_elems,
                   cast_at_use=not args.cast_on_copy, early_embedding_update=not args.no_early_embedding,
                   bf16_reload=False if args.no_bf16_reload else None, checkpoint_d2h=args.checkpoint_d2h,
                   h2d_issue_limit=args.h2d_issue_limit, **kw)
    uses_storage = args.ac_offload == "nvme" or args.opt_nvme_fraction > 0
    log(f"[bench] SlideFSDP ({h2d_format} H2D, {sf.resident_layers} resident decoders, {d2h_engine} D2H) "
        f"ready in {time.time() - t0:.1f}s")
    B, S = w["batch"], w["seq"]
    n_steps = args.steps if steps is None else steps
    n_warm = args.warmup if warmup is None else warmup
    g = torch.Generator().manual_seed(batch_seed)
    batches = [torch.randint(0, w["vocab"], (B, S), generator=g).to(dev) for _ in range(n_warm + n_steps)]

    for i in range(n_warm):
        t = time.time()
        out = sf(input_ids=batches[i], labels=batches[i])
        sf.wait_for_updates()
        torch.cuda.synchronize()
        log(f"[bench] warmup {i}: loss {out.loss.item():.4f} {time.time() - t:.2f}s")

    from test1_amd import kernels as _k

    rt = sf.runtime
    rt.stager.cast_timing, rt.stager.copy_timing, rt.d2h_timing = [], [], []
    rt.enable_link_timing(not args.no_link_timing)
    if rt.d2h_engine == "sdma":
        _k.dma_enable_timing(True)
    if timeline:
        rt.timeline = []
    io0 = _storage_snapshot(sf) if uses_storage else None
    # one clock for HIP events and SDMA copy times: an anchor event, and the
    # SDMA clock read right after the anchor has completed
    anchor = torch.cuda.Event(enable_timing=True)
    anchor.record()
    torch.cuda.synchronize()
    anchor_ns = _k.dma_clock_ns() if rt.d2h_engine == "sdma" else 0
    t_start = time.perf_counter()
    losses = []
    for i in range(n_steps):
        out = sf(input_ids=batches[n_warm + i], labels=batches[n_warm + i])
        losses.append(out.loss)
        log(f"[bench] step {i} issued")
    sf.wait_for_updates()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t_start
    losses = [x.item() for x in losses]
    if not all(math.isfinite(x) for x in losses):
        log(f"[bench] WARNING: non-finite training losses {losses}: the step's results are wrong")
    if timeline:
        with open(timeline, "w") as f:
            for t, th, what, unit in rt.timeline:
                f.write(f"{(t - t_start) * 1e3:.3f} {th} {what} {unit}\n")
    log(f"[bench] timed {n_steps} steps in {elapsed:.2f}s, losses {losses}")
    storage_stats = None
    if uses_storage:
        io1 = _storage_snapshot(sf)
        storage_stats = {k: io1[k] - io0[k] for k in io1}
        rd, wr, busy = storage_stats["bytes_read"], storage_stats["bytes_written"], storage_stats["busy_s"]
        storage_stats.update({
            "read_bytes_per_step": rd / n_steps, "write_bytes_per_step": wr / n_steps,
            "busy_frac": busy / elapsed, "gbs_while_busy": (rd + wr) / busy / 1e9 if busy > 0 else None})
        log(f"[bench] storage: {storage_stats}")
    link = link_timeline(rt, anchor, anchor_ns)
    h2d_idle = None
    if timeline and link["common_clock"]:
        h2d_idle = h2d_idle_attribution([(t - t_start, th, what, u) for t, th, what, u in rt.timeline], link,
                                        anchor_ns, elapsed)
        log(f"[bench] H2D idle: {h2d_idle}")
    if timeline:
        # the host-link and compute intervals on the host timeline's clock
        # (ms since the first timed step; the SDMA clock was read at t_start)
        with open(timeline + ".link.json", "w") as f:
            json.dump({d: {k: [((a - anchor_ns) * 1e-6, (b - anchor_ns) * 1e-6, n) for a, b, n in v]
                           for k, v in link[d].items()} for d in ("h2d", "d2h")}
                      | {"compute": [((a - anchor_ns) * 1e-6, (b - anchor_ns) * 1e-6) for a, b in link["compute"]],
                         "elapsed_ms": elapsed * 1e3, "steps": n_steps}, f)
    r = {
        "elapsed": elapsed, "losses": losses, "tokens": B * S * n_steps, "steps": n_steps, "warmup": n_warm,
        "cast": elapsed_stats(rt.stager.cast_timing), "ncast": len(rt.stager.cast_timing or []),
        "h2d": elapsed_stats(rt.stager.copy_timing), "d2h": elapsed_stats(rt.d2h_timing),
        "link": link, "h2d_idle": h2d_idle,
        "total_params": sf.total_params, "resident_layers": sf.resident_layers,
        "stage_after_update": sf.runtime.stage_after_update,
        "cast_at_use": sf.runtime.cast_at_use,
        "row_sparse_embedding": sf.layer_states[0].row_sparse,
        "bf16_reload_units": len(sf.bf16_reload_units),
        "layer_numel": sum(p.numel() for p in sf.decoder_layers[0].parameters()),
        "output_numel": sum(p.numel() for p in sf.output_layer.parameters()),
        "storage": storage_stats,
    }
    if after is not None:
        r["after"] = after(sf)
    sf.close()
    # The parameters point at the wrapper's pinned masters; give them pageable
    # copies, so the pinned memory goes with the wrapper (a next wrapper on
    # this model pins its own, and the driver caps pinned memory per process).
    with torch.no_grad():
        for p in model.parameters():
            p.data = p.data.clone()
    del sf, out, rt
    gc.collect()
    # The device memory stays in torch's cache for the next run (the next
    # wrapper reuses it; on a shortage the allocator frees it itself).  After
    # an empty_cache() that followed a SlideFSDP run, the activation round
    # trip's host-to-device copies ran at 44 GB/s against 55 without (the
    # cause was not found), so no measurement here empties the cache.
    return r


def cast_alone(dev, n: int, reps: int = 20, pairs: int = 4) -> dict:
    """The staging cast on an otherwise idle GPU, for context beside the
    in-pipeline figure: ``n``-element launches (after 3 warmups) on a stream
    of their own, timed with HIP events stamped around the kernel as in the
    pipeline figure.  The launches cycle through ``pairs`` source/destination
    pairs (6 B x n each, 5 GB for a Llama-3-8B layer and 4 pairs), so that no
    launch finds its operands in the 256 MB Infinity Cache."""
    import torch

    from test1_amd import kernels

    bufs = [(torch.randn(n, device=dev), torch.empty(n, dtype=torch.bfloat16, device=dev)) for _ in range(pairs)]
    st = torch.cuda.Stream(device=dev)
    for k in range(3):
        src, dst = bufs[k % pairs]
        kernels.cast_f32_bf16_(dst, src, st)
    timers = [kernels.KernelTimer() for _ in range(reps)]
    for k, t in enumerate(timers):
        src, dst = bufs[k % pairs]
        kernels.cast_f32_bf16_(dst, src, st, timer=t)
    st.synchronize()
    ms = sum(t.elapsed_ms() for t in timers) / reps
    gbs = 6 * n / (ms * 1e-3) / 1e9
    del bufs
    return {"elements": n, "launches": reps, "operand_pairs": pairs, "avg_launch_ms": ms, "achieved": gbs,
            "frac": gbs / HBM_PEAK_GBS}


def _storage_snapshot(sf) -> dict:
    """Counters of the storage engine and of the two offloaders' waits."""
    from test1_amd import storage

    st = storage.default_engine().stats()
    off = sf.layer_optimizer.offloader
    spill = sf._spill
    return {"bytes_read": st["bytes_read"], "bytes_written": st["bytes_written"], "busy_s": st["busy_s"],
            "bytes_staged": st["bytes_staged"],
            "optimizer_wait_s": 0.0 if off is None else off.wait_s,
            "checkpoint_slot_wait_s": 0.0 if spill is None else spill.slot_wait_s}


def variant_summary(v: dict, h2d_format: str, d2h_engine: str, alone: Optional[dict] = None) -> dict:
    cast_ms, cast_elems = v["cast"]
    cast_gbs = 6 * cast_elems / (cast_ms * 1e-3) / 1e9 if cast_ms > 0 else None
    return {"value": v["tokens"] / v["elapsed"], "ms_per_step": v["elapsed"] / v["steps"] * 1e3,
            "steps": v["steps"], "warmup": v["warmup"], "h2d_format": h2d_format,
            "resident_layers": v["resident_layers"], "d2h_engine": d2h_engine,
            "bf16_reload_units": v["bf16_reload_units"],
            "cast_frac": None if cast_gbs is None else cast_gbs / HBM_PEAK_GBS,
            "host_link": link_stats(v, v["steps"], alone), "losses": v["losses"],
            "losses_finite": all(math.isfinite(x) for x in v["losses"])}


def megatron_flops_per_step(w: dict) -> float:
    """Model FLOPs of one training step by the Megatron-LM estimate with GQA
    and SwiGLU that the reference reports (utils/metric.py:4-53): 3 passes x
    2 FLOPs per multiply-add x 2 (forward GEMM pairs), no recompute term."""
    B, S, L, H = w["batch"], w["seq"], w["layers"], w["hidden"]
    heads, kv, inter, vocab = w["heads"], w["kv"], w["inter"], w["vocab"]
    q_ratio = (H // heads) * heads / H
    attention = (1 + kv / heads + S / H) * q_ratio
    mlp = inter / H * 1.5
    logits = vocab / (2 * L * H)
    return 12.0 * B * S * L * H * H * (attention + mlp + logits)


def host_dram_stats(r: dict, args, cpu: Optional[dict]) -> dict:
    """Host DRAM traffic of one step: the host AdamW's 26 B per parameter
    (28 with the bf16 copy) plus every host-link transfer, each of which
    reads or writes host memory once (parameter copies, checkpoints and
    embedding rows both ways; gradient copies without engine timestamps
    included).  The reference rate is a streaming AdamW on the same cores in
    the same run (the CPU baseline's), the nearest this host gets to its
    DRAM peak."""
    adam_b = (28 if args.h2d_format == "bf16" else 26) * r["total_params"]
    lk = r.get("link") or {}
    link_b = sum(sp[2] for d in ("h2d", "d2h") for v in (lk.get(d) or {}).values() for sp in v)
    link_b += lk.get("untimed_d2h_bytes", 0)
    if link_b == 0:
        link_b = r["h2d"][1] + r["d2h"][1]
    step_s = r["elapsed"] / args.steps
    total = adam_b + link_b / args.steps
    ref = None if cpu is None else cpu.get("adam_gbs")
    return {"bytes_per_step": total, "adam_bytes_per_step": adam_b, "achieved_gbs": total / step_s / 1e9,
            "streaming_adam_gbs": ref, "frac_of_streaming_adam": None if not ref else total / step_s / 1e9 / ref}


def host_mem_available() -> int:
    """MemAvailable of this host in bytes (0 if unknown)."""
    try:
        for line in open("/proc/meminfo"):
            if line.startswith("MemAvailable:"):
                return int(line.split()[1]) * 1024
    except OSError:
        pass
    return 0


def link_timeline(rt, anchor, anchor_ns: int) -> dict:
    """Every host-link transfer and every unit's compute of the timed steps as
    (start_ns, end_ns[, bytes]) on one clock: HIP events placed by their time
    since ``anchor`` (recorded and completed at ``anchor_ns`` of the SDMA
    clock), SDMA gradient copies by their engine timestamps.
    h2d: parameter copies, checkpoint prefetches, embedding lookup rows read
    from the host table; d2h: gradient copies, checkpoint packs, embedding
    gradient rows."""
    def ns(ev):
        return anchor_ns + anchor.elapsed_time(ev) * 1e6

    def spans(records):
        out = []
        for rec in records or []:
            if _untimed(rec):
                continue
            if len(rec) == 4:                      # ("interval_ns", start, end, bytes)
                out.append((rec[1], rec[2], rec[3]))
            else:                                  # (start event, end event, bytes)
                out.append((ns(rec[0]), ns(rec[1]), rec[2]))
        return out

    lt = rt.link_timing or {}
    return {
        "h2d": {"params": spans(rt.stager.copy_timing), "checkpoints": spans(lt.get("act_h2d")),
                "rows": spans(lt.get("rows_h2d"))},
        "d2h": {"grads": spans(rt.d2h_timing), "checkpoints": spans(lt.get("act_d2h")),
                "rows": spans(lt.get("rows_d2h"))},
        "compute": [(ns(a), ns(b)) for a, b in lt.get("compute", [])],
        "common_clock": anchor_ns != 0,
        "untimed_d2h_bytes": sum(rec[1] for rec in list(rt.d2h_timing or []) + list(lt.get("act_d2h") or [])
                                 if _untimed(rec)),
    }


def h2d_idle_attribution(events, link: dict, anchor_ns: int, elapsed_s: float) -> dict:
    """Where the H2D direction idles in the timed steps: each gap between
    its transfers (parameter copies, checkpoint prefetches, lookup rows) is
    attributed to what the copy that ends it waited for.  ``events`` is the
    host timeline (perf_counter seconds since the first timed step, thread,
    event, unit); a copy whose issue (``staged_after_update`` by the update
    thread, ``h2d_issued`` by the forward) came less than 1 ms before it
    started waited for the host to issue it; one issued earlier waited on the
    device (its stream's order or an event)."""
    spans = sorted(((a - anchor_ns) * 1e-6, (b - anchor_ns) * 1e-6) for v in link["h2d"].values() for a, b, _ in v)
    union = []
    for a, b in spans:
        if union and a <= union[-1][1]:
            union[-1][1] = max(union[-1][1], b)
        else:
            union.append([a, b])
    total = elapsed_s * 1e3
    issues = sorted((t * 1e3, what) for t, _, what, _ in events if what in ("staged_after_update", "h2d_issued"))
    out = {"window_ms": total, "idle_ms": 0.0, "waiting_on_device_ms": 0.0, "waiting_for_update_thread_ms": 0.0,
           "waiting_for_forward_ms": 0.0, "gaps": 0}
    import bisect

    times = [t for t, _ in issues]
    prev_end = 0.0
    for a, b in union + [[total, total]]:
        gap = min(a, total) - prev_end
        prev_end = max(prev_end, b)
        if gap <= 0:
            continue
        out["gaps"] += 1
        out["idle_ms"] += gap
        k = bisect.bisect_right(times, a + 0.05) - 1
        if a >= total - 1e-6:
            continue
        if k >= 0 and a - times[k] < 1.0:
            key = "waiting_for_update_thread_ms" if issues[k][1] == "staged_after_update" else "waiting_for_forward_ms"
        else:
            key = "waiting_on_device_ms"
        out[key] += gap
    out["idle_frac"] = out["idle_ms"] / total if total > 0 else None
    return out


def _union(spans):
    """Sorted disjoint (start, end) covering the given spans."""
    out = []
    for s, e in sorted((sp[0], sp[1]) for sp in spans):
        if out and s <= out[-1][1]:
            out[-1][1] = max(out[-1][1], e)
        else:
            out.append([s, e])
    return out


def _length(u):
    return sum(e - s for s, e in u)


def _overlap(a, b):
    """Length of the intersection of two sorted disjoint interval lists."""
    i = j = 0
    tot = 0.0
    while i < len(a) and j < len(b):
        lo, hi = max(a[i][0], b[j][0]), min(a[i][1], b[j][1])
        if hi > lo:
            tot += hi - lo
        if a[i][1] < b[j][1]:
            i += 1
        else:
            j += 1
    return tot


def link_stats(r: dict, steps: int, alone: Optional[dict] = None) -> dict:
    """Per direction: bytes per step, the time per step at least one transfer
    of that direction was in flight (union of their intervals), the rate
    while busy against the nominal and the measured plain-copy peak, and the
    fraction of that busy time during which the compute stream was running a
    unit's forward or backward."""
    lk = r["link"]
    comp = _union(lk["compute"])
    out = {"peak_gbs": LINK_PEAK_GBS, "alone": alone}
    unions = {d: _union([sp for v in lk[d].values() for sp in v]) for d in ("h2d", "d2h")}
    duplex = (alone or {}).get("duplex")
    for d in ("h2d", "d2h"):
        parts = lk[d]
        allsp = [sp for v in parts.values() for sp in v]
        u = unions[d]
        busy_ns = _length(u)
        both_ns = _overlap(u, unions["d2h" if d == "h2d" else "h2d"])
        nbytes = sum(sp[2] for sp in allsp)
        gbs = nbytes / busy_ns if busy_ns > 0 else None
        measured = None if not alone else alone.get(f"{d}_gbs")
        # What plain copies would move in the same busy time: the duplex
        # copy's rate while the other direction is busy too, the one-way
        # copy's rate while it is not.
        model_bytes = None
        dup = (duplex or {}).get(f"{d}_gbs")
        if measured and dup and busy_ns > 0:
            model_bytes = both_ns * dup + (busy_ns - both_ns) * measured
        out[d] = {
            "bytes_per_step": nbytes / steps,
            "bytes_per_step_by_kind": {k: sum(sp[2] for sp in v) / steps for k, v in parts.items()},
            "busy_ms_per_step": busy_ns / steps * 1e-6,
            "both_directions_busy_ms_per_step": both_ns / steps * 1e-6,
            "gbs_while_busy": gbs,
            "frac": None if gbs is None else gbs / LINK_PEAK_GBS,
            "frac_of_measured_copy": None if gbs is None or not measured else gbs / measured,
            "frac_of_duplex_copy": None if gbs is None or not dup else gbs / dup,
            "frac_of_copy_model": None if not model_bytes else nbytes / model_bytes,
            "busy_frac_of_step": busy_ns * 1e-9 / r["elapsed"],
            "under_compute_frac": (_overlap(u, comp) / busy_ns) if (busy_ns > 0 and lk["common_clock"]) else None,
        }
        untimed = lk.get(f"untimed_{d}_bytes", 0)
        if untimed:
            out[d]["untimed_bytes_per_step"] = untimed / steps
            out[d]["untimed_note"] = ("SDMA copies (gradients, checkpoints) without engine timestamps (a profiler "
                                      "tracing async copies takes them over): the rates above cover the timed "
                                      "transfers only")
    out["compute_busy_frac_of_step"] = _length(comp) * 1e-9 / r["elapsed"]
    out["note"] = ("rates over the union of all transfers of a direction (h2d: parameter copies, checkpoint "
                   "prefetches, embedding lookup rows; d2h: SDMA gradient copies, checkpoint packs, embedding "
                   "gradient rows), HIP events and SDMA engine timestamps on one clock; under_compute_frac: "
                   "share of that time while the compute stream ran a unit's forward or backward (events "
                   "at unit boundaries, after the stream's waits for the unit's weights and checkpoint; gaps "
                   "between a unit's kernels count as compute); alone: plain pinned copies of 1 GiB, one "
                   "direction at a time, and (duplex) both directions at once; frac_of_copy_model: bytes moved "
                   "over what plain copies would move in the same busy time (the duplex rate while the other "
                   "direction is busy, the one-way rate otherwise)")
    return out


def link_alone(dev, nbytes: int = 1 << 30, reps: int = 4) -> dict:
    """Plain pinned-host <-> device copies of ``nbytes``, one direction at a
    time on an idle GPU: the host link rate this box reaches."""
    import torch

    from test1_amd.pinned import pinned_empty

    host = pinned_empty(nbytes, torch.uint8)
    host.fill_(1)
    devbuf = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    st = torch.cuda.Stream(device=dev)
    out = {}
    for d, (dst, src) in (("h2d", (devbuf, host)), ("d2h", (host, devbuf))):
        with torch.cuda.stream(st):
            dst.copy_(src, non_blocking=True)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(st)
        with torch.cuda.stream(st):
            for _ in range(reps):
                dst.copy_(src, non_blocking=True)
        e1.record(st)
        st.synchronize()
        out[f"{d}_gbs"] = nbytes * reps / (e0.elapsed_time(e1) * 1e-3) / 1e9
    del host, devbuf
    return out


def link_kernels_alone(dev, w: dict, reps: int = 10) -> dict:
    """The host-link kernels of the step on an otherwise idle GPU, at the
    step's shapes: the embedding lookup (batch rows of a pinned fp32 table
    of the vocabulary's size, cast to bf16), the gradient rows and the
    checkpoint pack (bf16 into pinned host memory, the runtime's 16 workgroups).  Average
    ms per launch (HIP events around each launch, 3 warmups) and GB/s of
    link bytes."""
    import torch

    from test1_amd import kernels
    from test1_amd.pinned import pinned_empty

    V, H, ntok = w["vocab"], w["hidden"], w["batch"] * w["seq"]
    g = torch.Generator().manual_seed(3)
    ids = torch.randint(0, V, (ntok,), generator=g).to(dev)
    table = pinned_empty((V, H), torch.float32)
    table.fill_(0.5)
    rows_dev = torch.empty(ntok, H, dtype=torch.bfloat16, device=dev)
    dense = torch.zeros(V, H, dtype=torch.bfloat16, device=dev)
    rows_host = pinned_empty((ntok, H), torch.bfloat16)
    act = torch.zeros(w["batch"], w["seq"], H, dtype=torch.bfloat16, device=dev)
    act_host = pinned_empty(tuple(act.shape), torch.bfloat16)
    st = torch.cuda.Stream(device=dev)
    cases = {
        "gather_rows_kernel<cast>": (lambda: kernels.gather_rows(table, ids, rows_dev, stream=st), ntok * H * 4),
        "gather_rows_kernel<copy> (16 workgroups)": (
            lambda: kernels.gather_rows(dense, ids, rows_host, stream=st, max_workgroups=D2H_WORKGROUPS), ntok * H * 2),
        "seg_kernel<OpCopy16> (16 workgroups)": (
            lambda: kernels.copy_segs_b16([(act.view(-1), act_host.view(-1))], st, max_workgroups=D2H_WORKGROUPS),
            act.numel() * 2),
    }
    out = {}
    for name, (fn, nbytes) in cases.items():
        for _ in range(3):
            fn()
        evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(reps)]
        for a, b in evs:
            a.record(st)
            fn()
            b.record(st)
        st.synchronize()
        ms = sum(a.elapsed_time(b) for a, b in evs) / reps
        out[name] = {"avg_launch_ms": ms, "achieved": nbytes / (ms * 1e-3) / 1e9,
                     "frac": nbytes / (ms * 1e-3) / 1e9 / LINK_PEAK_GBS}
    del table, dense, rows_host, act_host
    return out


def _ms_spans(anchor, pairs):
    """(start, end) in ms since ``anchor`` of (start_event, end_event) pairs."""
    return [(anchor.elapsed_time(a), anchor.elapsed_time(b)) for a, b in pairs]


def param_streaming(sf, dev, passes: int = 3, seq: int = 1024) -> dict:
    """The parameter-streaming configuration on a wrapper with every unit in
    the 2-unit pool: its decoder layers streamed forward-only, the next
    layer's load (pinned fp32 master -> device slot, cast to bf16 where it is
    used) issued before each layer's forward (reference slide_fsdp.py:363-409,
    layer_state.py:273-328), on [1, seq, hidden] bf16 N(0, 1) hidden states.
    One warmup pass, then ``passes`` timed passes between device
    synchronisations.  Reports the H2D rate over the pass and while busy, the
    staging cast against HBM peak, and how copies and layer compute overlap."""
    import torch

    rt = sf.runtime
    sf.release_device_units()
    states = sf.layer_states[1:-1]
    H = sf.model_config.hidden_size
    h0 = torch.randn(1, seq, H, generator=torch.Generator(device=dev).manual_seed(42), device=dev).bfloat16()
    pos = sf.rotary_emb(h0, torch.arange(seq, device=dev).unsqueeze(0))
    comp = torch.cuda.current_stream()
    compute = []

    def one_pass(record: bool):
        h = h0
        states[0].to_device_async()
        for i, st in enumerate(states):
            if i + 1 < len(states):
                states[i + 1].to_device_async()   # prefetch the next layer
            st.wait_for_h2d()
            if record:
                a = torch.cuda.Event(enable_timing=True)
                a.record(comp)
            with torch.no_grad():
                out = st.layer(h, attention_mask=None, position_embeddings=pos, use_cache=False)
            h = out[0] if isinstance(out, (tuple, list)) else out
            if record:
                b = torch.cuda.Event(enable_timing=True)
                b.record(comp)
                compute.append((a, b))
            st.to_offload_async(is_backward=False)
        return h

    one_pass(False)
    torch.cuda.synchronize()
    rt.stager.copy_timing, rt.stager.cast_timing = [], []
    anchor = torch.cuda.Event(enable_timing=True)
    anchor.record(comp)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(passes):
        h = one_pass(True)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    finite = bool(torch.isfinite(h.float()).all())
    copies = [(anchor.elapsed_time(a), anchor.elapsed_time(b), n) for a, b, n in rt.stager.copy_timing]
    nbytes = sum(n for _, _, n in copies)
    u_h2d = _union(copies)
    u_comp = _union(_ms_spans(anchor, compute))
    busy_ms, comp_ms = _length(u_h2d), _length(u_comp)
    both_ms = _overlap(u_h2d, u_comp)
    cast_ms, cast_elems = elapsed_stats(rt.stager.cast_timing)
    ncast = len(rt.stager.cast_timing)
    cast_gbs = 6 * cast_elems / (cast_ms * 1e-3) / 1e9 if cast_ms > 0 else None
    rt.stager.copy_timing = rt.stager.cast_timing = None
    gbs = nbytes / wall / 1e9
    busy_gbs = nbytes / (busy_ms * 1e-3) / 1e9 if busy_ms > 0 else None
    return {
        "workload": (f"{len(states)} decoder layers ({states[0].total_size:,} fp32 parameters each, pinned) "
                     f"streamed forward-only through the 2-unit pool, next layer's load issued before each "
                     f"forward, [1, {seq}, {H}] bf16 N(0,1) input"),
        "value": gbs, "unit": "GB/s (H2D over the whole pass)", "passes": passes,
        "ms_per_pass": wall / passes * 1e3, "h2d_bytes_per_pass": nbytes / passes,
        "h2d_gbs_while_busy": busy_gbs, "frac": gbs / LINK_PEAK_GBS,
        "frac_while_busy": None if busy_gbs is None else busy_gbs / LINK_PEAK_GBS,
        "h2d_busy_frac_of_pass": busy_ms * 1e-3 / wall,
        "cast": {"kernel": "cast_flat_kernel", "launches": ncast,
                 "avg_launch_ms": cast_ms / ncast if ncast else None, "achieved": cast_gbs, "peak": HBM_PEAK_GBS,
                 "unit": "GB/s", "frac": None if cast_gbs is None else cast_gbs / HBM_PEAK_GBS},
        "compute_ms_per_pass": comp_ms / passes,
        "compute_under_h2d_frac": both_ms / comp_ms if comp_ms > 0 else None,
        "h2d_under_compute_frac": both_ms / busy_ms if busy_ms > 0 else None,
        "output_finite": finite,
        "note": ("value: H2D bytes / wall time of the passes; compute_under_h2d_frac: share of the layers' "
                 "forward time during which a parameter copy was in flight (the prefetch hidden behind the "
                 "forward); with [1, 1024] tokens a layer computes in ~1 ms against ~16 ms for its copy, so "
                 "the pass is bound by the host link"),
    }


def activation_round_trip(dev, L: int = 32, shape=(4, 1024, 4096), rounds: int = 4, warmup: int = 2) -> dict:
    """The activation-offload configuration: ``L`` checkpointed layers whose
    bf16 inputs of ``shape`` (N(0,1)) go to pinned host slots through
    ``SlidingCheckpoint`` in the forward (SDMA copies, as SlideFSDP makes
    them with its default engines) and come back one layer ahead in the
    backward (prefetch on the H2D stream,
    reference sliding_checkpoint.py:51-131), on the runtime's streams.  The layers compute an
    elementwise ``tanh(x) * w``, so the copies dominate.  The first
    ``warmup`` rounds are not timed (in a fresh process the first call's
    H2D ran at 46.9 GB/s after one warmup round, later calls at 51-53); the
    last round also checks that every recompute was given its forward input
    bit for bit.  Reports each direction's rate over the union of its
    transfers against the nominal link."""
    import torch
    from torch.utils.checkpoint import checkpoint

    from test1_amd import kernels as _k
    from test1_amd.layer_state import runtime_streams
    from test1_amd.pinned import pinned_empty
    from test1_amd.sliding_checkpoint import ActivationRing, SlidingCheckpoint

    _k.dma_init(dev)
    _k.dma_enable_timing(True)
    slots = [[pinned_empty(shape, torch.bfloat16)] for _ in range(L)]
    # the streams SlideFSDP gives the checkpoint offload and its prefetch
    h2d, _, d2h = runtime_streams(dev)
    ws = [torch.full((shape[-1],), 1.0 + 1e-3 * i, dtype=torch.bfloat16, device=dev, requires_grad=True)
          for i in range(L)]
    h = torch.randn(shape, generator=torch.Generator(device=dev).manual_seed(42), device=dev).bfloat16()
    h.requires_grad_(True)
    ring = ActivationRing(dev)

    def layer_fn(x, w):
        return torch.tanh(x) * w

    out = {}
    fwd_ms = bwd_ms = 0.0
    d2h_sp, h2d_sp = [], []
    exact = None
    comp = torch.cuda.current_stream()
    for rnd in range(rounds):
        lt = {"act_d2h": [], "act_h2d": []}
        check = rnd == rounds - 1
        served = {} if check else None
        inputs = []
        anchor = torch.cuda.Event(enable_timing=True)
        anchor.record(comp)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        x = h
        for i in range(L):
            if check:
                inputs.append(x.detach())
            with SlidingCheckpoint(layer_idx=i + 1, layer_tensors=slots, is_last_layer=(i == L - 1), no_mask=True,
                                   device=str(dev), stream=d2h, prefetch_stream=h2d, prefetch_ring=ring,
                                   link_timing=lt, served=served, pack_engine="sdma"):
                x = checkpoint(layer_fn, x, ws[i], use_reentrant=False)
        loss = x.float().sum()
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        loss.backward()
        torch.cuda.synchronize()
        t2 = time.perf_counter()
        for w in ws:
            w.grad = None
        h.grad = None
        if rnd < warmup:
            continue
        fwd_ms += (t1 - t0) * 1e3
        bwd_ms += (t2 - t1) * 1e3
        # SDMA copies: engine timestamps (ns of the system clock)
        d2h_sp += [(rec[1] * 1e-6, rec[2] * 1e-6, rec[3]) for rec in lt["act_d2h"] if rec[0] == "interval_ns"]
        h2d_sp += [(anchor.elapsed_time(a) + 1e6 * rnd, anchor.elapsed_time(b) + 1e6 * rnd, n)
                   for a, b, n in lt["act_h2d"]]
        if check:
            exact = all(torch.equal(served[(i, 0)].view(torch.int16), inputs[i].view(torch.int16))
                        for i in range(L))
            del served, inputs
    timed = rounds - warmup
    for d, sp in (("d2h", d2h_sp), ("h2d", h2d_sp)):
        nb = sum(n for _, _, n in sp)
        busy = _length(_union(sp))
        gbs = nb / (busy * 1e-3) / 1e9 if busy > 0 else None
        out[d] = {"bytes_per_round": nb / timed, "transfers_per_round": len(sp) / timed,
                  "busy_ms_per_round": busy / timed, "gbs_while_busy": gbs,
                  "frac": None if gbs is None else gbs / LINK_PEAK_GBS}
    ring.close()
    del slots
    per_layer = 2 * math.prod(shape)
    return {
        "workload": (f"{L} layers x bf16 {list(shape)} N(0,1) checkpoints ({per_layer:,} B each) packed to pinned "
                     f"host slots in the forward and prefetched back one layer ahead in the backward "
                     f"(the last layer keeps its checkpoint on the GPU)"),
        "value": None if out["h2d"]["gbs_while_busy"] is None else min(out["h2d"]["gbs_while_busy"],
                                                                        out["d2h"]["gbs_while_busy"] or 0.0),
        "unit": "GB/s (the slower direction, while busy)", "rounds_timed": timed,
        "forward_ms_per_round": fwd_ms / timed, "backward_ms_per_round": bwd_ms / timed,
        "d2h": out["d2h"], "h2d": out["h2d"], "bit_exact": exact,
        "note": ("d2h: SDMA copies (ROCr, engine 3) into the pinned slots, started by the ring's worker "
                 "thread; h2d: hipMemcpyAsync of each slot into a 2-set device ring; rates over the union of "
                 "each direction's transfer intervals (engine timestamps, HIP events on the H2D stream)"),
    }


def link_duplex(dev, nbytes: int = 1 << 30, reps: int = 4) -> dict:
    """Both directions at once, with the step's own copy paths: ``reps``
    host-to-device copies of ``nbytes`` (hipMemcpyAsync on a stream, as the
    parameter copies) and, issued right behind them, ``reps`` device-to-host
    copies of ``nbytes`` on the SDMA engines of the gradient copies.  Each
    direction's rate over its own span (HIP events; SDMA engine timestamps),
    and the share of the device-to-host span the host-to-device copies
    covered: the rate each direction keeps while the other is busy."""
    import torch

    from test1_amd import kernels
    from test1_amd.pinned import pinned_empty

    kernels.dma_init(dev)
    kernels.dma_enable_timing(True)
    h_src = pinned_empty(nbytes, torch.uint8)
    h_dst = pinned_empty(reps * nbytes, torch.uint8)
    h_src.fill_(1)
    d_dst = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    d_src = torch.ones(nbytes, dtype=torch.uint8, device=dev)
    up = torch.cuda.Stream(device=dev)
    with torch.cuda.stream(up):
        d_dst.copy_(h_src, non_blocking=True)
    kernels.DmaReady(kernels.dma_copy_d2h([(d_src, h_dst[:nbytes])]), timeout=60).release()
    torch.cuda.synchronize()
    anchor = torch.cuda.Event(enable_timing=True)
    anchor.record(up)
    anchor.synchronize()
    anchor_ns = kernels.dma_clock_ns()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(up)
    with torch.cuda.stream(up):
        for _ in range(reps):
            d_dst.copy_(h_src, non_blocking=True)
    e1.record(up)
    handle = kernels.dma_copy_d2h([(d_src, h_dst[k * nbytes:(k + 1) * nbytes]) for k in range(reps)])
    t0, t1 = kernels.DmaReady(handle, timeout=60).release()
    torch.cuda.synchronize()
    h2d_s = (anchor_ns + anchor.elapsed_time(e0) * 1e6, anchor_ns + anchor.elapsed_time(e1) * 1e6)
    out = {"h2d_gbs": nbytes * reps / ((h2d_s[1] - h2d_s[0]) * 1e-9) / 1e9}
    if t1 > t0:
        out["d2h_gbs"] = nbytes * reps / ((t1 - t0) * 1e-9) / 1e9
        out["d2h_span_under_h2d_frac"] = max(0.0, min(t1, h2d_s[1]) - max(t0, h2d_s[0])) / (t1 - t0)
        out["aggregate_gbs"] = out["h2d_gbs"] + out["d2h_gbs"]
    out["note"] = ("host-to-device: hipMemcpyAsync on a stream; device-to-host: the gradient copies' SDMA "
                   "engines, issued right after; each rate over its own span")
    del h_src, h_dst, d_dst, d_src
    return out


def run_child_workload(workload: str, steps: int, warmup: int, env_hw_queues: Optional[str],
                       timeout_s: float = 900.0) -> dict:
    """Run this bench for another workload in a child process (its own
    pinned-memory budget and the environment's hardware queues) and return
    its JSON line's main figures, or ``{"skipped": reason}``."""
    import subprocess

    cmd = [sys.executable, "-u", os.path.abspath(__file__), "--workload", workload, "--steps", str(steps),
           "--warmup", str(warmup), "--no-variants", "--no-cpu-baseline", "--no-configs", "--hw-queues", "0"]
    env = dict(os.environ)
    if env_hw_queues is None:
        env.pop("GPU_MAX_HW_QUEUES", None)
    else:
        env["GPU_MAX_HW_QUEUES"] = env_hw_queues
    log(f"[bench] child run: {' '.join(cmd[2:])}")
    try:
        p = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=None, env=env, timeout=timeout_s, text=True)
    except subprocess.TimeoutExpired:
        return {"skipped": f"child run did not finish within {timeout_s:.0f} s"}
    lines = [ln for ln in p.stdout.splitlines() if ln.startswith("{")]
    if p.returncode != 0 or not lines:
        return {"skipped": f"child run exited with status {p.returncode}"}
    d = json.loads(lines[-1])
    hl = d.get("host_link") or {}
    return {
        "workload": d["config"]["workload"], "model": workload, "value": d["value"], "unit": d["unit"],
        "ms_per_step": d["ms_per_step"], "steps": d["steps"], "warmup": d["warmup"],
        "global_batch": d["config"]["global_batch"], "seq_len": d["config"]["seq_len"],
        "resident_layers": d["config"]["resident_layers"], "hw_queues": d["config"]["hw_queues"],
        "roofline": {k: d["roofline"].get(k) for k in ("bound", "achieved", "peak", "unit", "frac", "launches",
                                                       "avg_launch_ms")},
        "host_link": {k: {kk: hl[k].get(kk) for kk in ("bytes_per_step", "gbs_while_busy", "frac",
                                                       "busy_frac_of_step", "under_compute_frac")}
                      for k in ("h2d", "d2h") if isinstance(hl.get(k), dict)},
        "losses_finite": d["losses_finite"], "command": " ".join(["python"] + cmd[2:]),
    }


def secondary_rooflines(r: dict, alone: Optional[dict] = None, checkpoint_d2h: str = "kernel") -> list:
    """Host-link-bound work besides the staging cast: achieved rate over its
    own intervals in the step (timing events around each launch on its
    stream, or an SDMA engine's timestamps; the link is shared with the
    copies running beside it) and, in ``alone``, on an idle GPU."""
    lk = r["link"]
    rows = []
    if checkpoint_d2h == "sdma":
        ckpt = ("checkpoints", "d2h", "SDMA copy (ROCr, engine 3)", "checkpoint copy: HBM -> pinned host slot")
    else:
        ckpt = ("checkpoints", "d2h", "seg_kernel<OpCopy16> (16 workgroups)", "checkpoint pack: HBM -> pinned host slot")
    for kind, d, kernel, what in (
            ckpt,
            ("rows", "h2d", "gather_rows_kernel<cast>", "embedding lookup: batch rows of the pinned fp32 host "
                                                          "table -> bf16 hidden states in HBM"),
            ("rows", "d2h", "gather_rows_kernel<copy> (16 workgroups)",
             "embedding gradient rows: HBM -> pinned host")):
        sp = lk[d].get(kind) or []
        if not sp:
            continue
        ms = sum(e - s for s, e, _ in sp) * 1e-6
        nb = sum(n for _, _, n in sp)
        gbs = nb / (ms * 1e-3) / 1e9 if ms > 0 else None
        rows.append({"kernel": kernel, "work": what, "bound": "host link", "launches": len(sp),
                     "avg_launch_ms": ms / len(sp), "link_bytes_per_launch": nb / len(sp), "achieved": gbs,
                     "peak": LINK_PEAK_GBS, "unit": "GB/s", "frac": None if gbs is None else gbs / LINK_PEAK_GBS,
                     "alone": None if not alone else alone.get(kernel)})
    return rows


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--workload", default="llama3-8b", choices=sorted(WORKLOADS))
    ap.add_argument("--layers", type=int, default=0, help="override the number of decoder layers")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-variants", action="store_true",
                    help="skip the shorter timed runs of the reference's pool schedule and the other H2D format")
    ap.add_argument("--no-configs", action="store_true",
                    help="skip the parameter-streaming and activation round-trip configurations and the "
                         "Qwen2.5-14B step in a child process")
    ap.add_argument("--timeline", default="", help="write the host timeline of the timed steps to this file")
    ap.add_argument("--d2h-engine", default="sdma", choices=("sdma", "kernel", "copy"),
                    help="gradient D2H by a capped pack kernel, by DMA copies, or on SDMA engines via ROCr")
    ap.add_argument("--h2d-format", default="fp32", choices=("fp32", "bf16"),
                    help="parameter H2D as fp32 masters + GPU cast, or as the host optimizer's bf16 copy")
    ap.add_argument("--resident-layers", type=int, default=None,
                    help="decoder layers kept on the GPU from their forward to their backward "
                         "(default: as many as fit in half of the free HBM)")
    ap.add_argument("--fused-ce", action="store_true",
                    help="chunked linear + cross entropy in the output unit (no [B,S,V] logits)")
    ap.add_argument("--no-activation-checkpoint", action="store_true",
                    help="keep every decoder's activations in HBM (needs every unit resident): no recompute")
    ap.add_argument("--ac-offload", default="cpu", choices=("cpu", "nvme", "none"),
                    help="checkpoint inputs to pinned host slots, to files on local storage, or kept on the GPU")
    ap.add_argument("--opt-nvme-fraction", type=float, default=0.0,
                    help="AdamW moments on local storage: exp_avg above 0, both moments above 0.5")
    ap.add_argument("--piece-elems", type=int, default=0,
                    help="elements per piece of a unit's update (gradients back, AdamW and copy to the device "
                         "run piece by piece, one cast per unit), e.g. 67108864; 0: whole units")
    ap.add_argument("--checkpoint-d2h", default=None, choices=("sdma", "kernel"),
                    help="how checkpoints reach their pinned slots (default: sdma with the sdma D2H engine)")
    ap.add_argument("--pool-size", type=int, default=2,
                    help="units in the device buffer pool (the reference's gpu_buffer_pool_size, default 2)")
    ap.add_argument("--h2d-issue-limit", type=int, default=3,
                    help="unit copies the forward and backward may keep queued before they wait (0: no limit)")
    ap.add_argument("--no-early-embedding", action="store_true",
                    help="update the embedding's untouched rows with its batch rows, after the backward, "
                         "instead of as the backward starts")
    ap.add_argument("--cast-on-copy", action="store_true",
                    help="cast a unit staged after its update on the cast stream as soon as its copy lands "
                         "(default: where the unit is next used, between the forward's kernels)")
    ap.add_argument("--no-bf16-reload", action="store_true",
                    help="units reloaded for their backward come back as fp32 + GPU cast instead of from the "
                         "bf16 copy their update writes")
    ap.add_argument("--hw-queues", type=int, default=None,
                    help="hardware queues of the HIP runtime (GPU_MAX_HW_QUEUES) for this process, set before "
                         "the first GPU call; 0 keeps the environment's.  Default: 8 for the Llama-3.1-8B "
                         "workload (the step drives four streams of its own beside torch's; with four queues two "
                         "of them share one, and the step ran 2.5 %% slower), the environment's otherwise: the "
                         "extra queues pin memory, and the fp32 Qwen2.5-14B step is at the pinned-memory limit")
    ap.add_argument("--wait-timeout", type=float, default=None,
                    help="seconds a host wait of the runtime may take (default: the library's; 0: no limit)")
    ap.add_argument("--no-link-timing", action="store_true",
                    help="do not record the host-link and compute intervals (no host_link figures)")
    ap.add_argument("--offload-dir", default="/tmp/sf_offload",
                    help="directory of the storage-offload files (removed as they are opened)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build runs the layer-streaming path on one GPU only; use --gpus 1", file=sys.stderr)
        sys.exit(2)

    # stdout carries the one JSON line only: everything else printed there
    # (the wrapper's model summary, the host AdamW's banner from C) goes to stderr.
    sys.stdout.flush()
    json_out = os.fdopen(os.dup(1), "w")
    os.dup2(2, 1)

    env_hw_queues = os.environ.get("GPU_MAX_HW_QUEUES")
    if args.hw_queues is None:
        args.hw_queues = 8 if args.workload == "llama3-8b" else 0
    if not 0 <= args.hw_queues <= 32:
        print("bench.py: --hw-queues must be in 0..32", file=sys.stderr)
        sys.exit(2)
    configs = {}
    if not args.no_configs and args.workload == "llama3-8b":
        # The Qwen2.5-14B step in a child process, run before this process
        # touches the GPU or builds its model: the child starts from a
        # process without a GPU context, and host memory and the driver's
        # pinned limit would not hold both models.
        avail = host_mem_available()
        if avail and avail < 200e9:
            configs["c5_qwen25_14b_step"] = {"skipped": f"needs ~200 GB of host memory, {avail / 1e9:.0f} GB available"}
        else:
            configs["c5_qwen25_14b_step"] = run_child_workload("qwen2.5-14b", 5, 2, env_hw_queues)
        log(f"[bench] Qwen2.5-14B step: {configs['c5_qwen25_14b_step']}")
    if args.hw_queues:
        # Read by the HIP runtime at its first call: set before torch touches the GPU.
        os.environ["GPU_MAX_HW_QUEUES"] = str(args.hw_queues)
    import torch

    w = dict(WORKLOADS[args.workload])
    if args.layers:
        w["layers"] = args.layers
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    t0 = time.time()
    model = build_model(w)
    log(f"[bench] model built in {time.time() - t0:.1f}s")
    B, S = w["batch"], w["seq"]

    r = timed_run(model, w, args, dev, args.h2d_format, args.resident_layers, args.d2h_engine, args.timeline)
    elapsed, losses = r["elapsed"], r["losses"]
    cast_ms, cast_elems = r["cast"]
    ncast = r["ncast"]
    cast_bytes = 6 * cast_elems  # read fp32 + write bf16 per element
    cast_gbs = cast_bytes / (cast_ms * 1e-3) / 1e9 if cast_ms > 0 else 0.0
    value = r["tokens"] / elapsed

    variants = {}
    raw_variants = {}
    if not args.no_variants:
        vs, vw = min(args.steps, 10), min(args.warmup, 2)
        # The reference's schedule: every unit in the 2-unit pool and reloaded
        # for its backward (slide_fsdp.py:443-444), for models whose bf16
        # weights do not fit in HBM.
        streaming = None if args.no_configs else (lambda sf: param_streaming(sf, dev))
        try:
            vp = timed_run(model, w, args, dev, args.h2d_format, 0, args.d2h_engine, batch_seed=2, steps=vs,
                           warmup=vw, after=streaming)
            raw_variants["pool"] = (vp, args.h2d_format, args.d2h_engine)
            if streaming is not None:
                configs["c2_param_streaming"] = vp["after"]
                log(f"[bench] parameter streaming: {vp['after']}")
        except RuntimeError as e:
            log(f"[bench] variant pool failed: {e}")
            variants["pool"] = {"skipped": str(e)[:300]}
        if args.h2d_format == "fp32":
            # the same schedule with the reference's link format: bf16 over the
            # link (here the host AdamW's bf16 copy, there a host cast at load time)
            try:
                vpb = timed_run(model, w, args, dev, "bf16", 0, args.d2h_engine, batch_seed=3, steps=vs,
                                warmup=vw)
                raw_variants["pool_bf16"] = (vpb, "bf16", args.d2h_engine)
            except RuntimeError as e:
                log(f"[bench] variant pool_bf16 failed: {e}")
                variants["pool_bf16"] = {"skipped": str(e)[:300]}
        # The other parameter H2D format, default residency.
        other = "bf16" if args.h2d_format == "fp32" else "fp32"
        # host bytes of the second wrapper: fp32 master, bf16 grad slot and two fp32
        # moments per parameter, plus the bf16 copy with bf16 H2D
        need = r["total_params"] * (4 + 2 + 8 + (2 if other == "bf16" else 0))
        avail = host_mem_available()
        if avail and need > 0.8 * avail:
            log(f"[bench] variant h2d_{other} skipped: needs ~{need / 1e9:.0f} GB of host memory, "
                f"{avail / 1e9:.0f} GB available")
            variants[f"h2d_{other}"] = {"skipped": f"needs ~{need / 1e9:.0f} GB host memory, "
                                                   f"{avail / 1e9:.0f} GB available"}
        else:
            try:
                v = timed_run(model, w, args, dev, other, args.resident_layers, args.d2h_engine, batch_seed=1,
                              steps=vs, warmup=vw)
                raw_variants[f"h2d_{other}"] = (v, other, args.d2h_engine)
            except RuntimeError as e:  # e.g. the host cannot pin the bf16 copies
                log(f"[bench] variant h2d_{other} failed: {e}")
                variants[f"h2d_{other}"] = {"skipped": str(e)[:300]}
    link_alone_gbs = link_alone(dev)
    log(f"[bench] plain pinned copies of 1 GiB: {link_alone_gbs}")
    duplex = link_duplex(dev)
    log(f"[bench] plain pinned copies of 1 GiB in both directions at once: {duplex}")
    link_alone_gbs["duplex"] = duplex
    for k, (v, fmt, eng) in raw_variants.items():
        variants[k] = variant_summary(v, fmt, eng, link_alone_gbs)
    variants = {k: variants[k] for k in ("pool", "pool_bf16", "h2d_bf16", "h2d_fp32") if k in variants}
    if not args.no_configs:
        configs["c3_activation_round_trip"] = activation_round_trip(dev, L=w["layers"], shape=(B, S, w["hidden"]))
        log(f"[bench] activation round trip: {configs['c3_activation_round_trip']}")
    kernels_alone = link_kernels_alone(dev, w)
    log(f"[bench] host-link kernels alone: {kernels_alone}")

    total_params = r["total_params"]
    layer_numel = r["layer_numel"]
    alone = cast_alone(dev, layer_numel)
    log(f"[bench] cast alone, one decoder layer: {alone['avg_launch_ms']:.4f} ms, {alone['achieved']:.0f} GB/s")
    resident = layer_numel + r["output_numel"]
    cpu = None
    if not args.no_cpu_baseline:
        t = time.time()
        cpu = cpu_baseline(total_params, B * S, resident)
        log(f"[bench] cpu baseline in {time.time() - t:.1f}s: {cpu['sample']}")

    res = {
        "metric": f"train tokens/s ({w['model']} layer offload, 1 GPU)",
        "value": value,
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": elapsed / args.steps * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (uniform random token ids, random-init N(0,0.02) weights)",
        "config": {"workload": f"{w['model']} causal-LM training step, fp32 masters in pinned host memory, "
                               f"layer-wise H2D ({args.h2d_format}"
                               f"{' + GPU RNE cast' if args.h2d_format == 'fp32' else ', host-cast in the AdamW pass'}), "
                               f"activation checkpoint offload, grad D2H, host LayerAdam",
                   "global_batch": B, "seq_len": S, "layers": w["layers"], "hidden": w["hidden"],
                   "params": total_params, "parallelism": "none (1 GPU)",
                   "h2d_format": args.h2d_format, "resident_layers": r["resident_layers"],
                   "hw_queues": int(os.environ.get("GPU_MAX_HW_QUEUES", "4")),
                   "d2h_engine": args.d2h_engine,
                   "checkpoint_d2h": args.checkpoint_d2h or ("sdma" if args.d2h_engine == "sdma" else "kernel"),
                   "fused_cross_entropy": args.fused_ce,
                   "stage_after_update": r["stage_after_update"],
                   "update_piece_elems": args.piece_elems, "h2d_issue_limit": args.h2d_issue_limit, "gpu_buffer_pool_size": args.pool_size,
                   "cast_at_use": r["cast_at_use"],
                   "bf16_reload_units": r["bf16_reload_units"],
                   "early_embedding_update": not args.no_early_embedding,
                   "row_sparse_embedding": r["row_sparse_embedding"],
                   "ac_offload_mode": args.ac_offload,
                   "activation_checkpoint": not args.no_activation_checkpoint,
                   "optimizer_nvme_offload_fraction": args.opt_nvme_fraction},
        "roofline": {
            "bound": "hbm",
            "kernel": "cast_flat_kernel (fp32 -> bf16 RNE staging cast)",
            "achieved": cast_gbs,
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": cast_gbs / HBM_PEAK_GBS,
            "traffic": (None if traffic_factor() is None or not ncast
                        else traffic_factor() * cast_bytes / ncast),
            "traffic_source": "profiles/cast_flat_kernel__pmc_llama3_8b_layer.md (FETCH_SIZE, WRITE_SIZE "
                              "scaled by a plain copy of known size)",
            "launches": ncast,
            "avg_launch_ms": cast_ms / ncast if ncast else None,
            "algorithmic_bytes_per_launch": cast_bytes / ncast if ncast else None,
            "alone": alone,
            "note": ("achieved/frac: every cast of the timed steps, "
                     + ("each on the forward's stream right before the unit's forward (units are copied "
                        "right after their update and cast where they are next used)"
                        if r["cast_at_use"] else
                        "most of them beside the backward's GEMMs (units are staged right after their "
                        "update)")
                     + "; alone: one decoder layer's cast on an idle GPU after the timed steps"),
        },
        "roofline_secondary": secondary_rooflines(
            r, kernels_alone, args.checkpoint_d2h or ("sdma" if args.d2h_engine == "sdma" else "kernel")),
        "host_link": dict(link_stats(r, args.steps, link_alone_gbs), h2d_idle=r["h2d_idle"]),
        "model_tflops": {
            "flops_per_step": megatron_flops_per_step(w),
            "tflops": megatron_flops_per_step(w) / (elapsed / args.steps) / 1e12,
            "note": "Megatron-LM estimate as the reference's utils/metric.py (no recompute term); "
                    "context only: the step is bound by the host link, not by MFMA",
        },
        "host_dram": host_dram_stats(r, args, cpu),
        "storage": r["storage"],
        "cpu_baseline": None if cpu is None else {k: cpu[k] for k in ("value", "unit", "cores", "kind", "sample")},
        "losses": losses,
        "losses_finite": all(math.isfinite(x) for x in losses),
        "variants": variants,
        "configs": {"c1_cpu_reference": "cpu_baseline", "c2_param_streaming": configs.get("c2_param_streaming"),
                    "c3_activation_round_trip": configs.get("c3_activation_round_trip"),
                    "c4_llama31_8b_step": "value (this line's headline)" if args.workload == "llama3-8b" else None,
                    "c5_qwen25_14b_step": configs.get("c5_qwen25_14b_step")},
    }
    print(json.dumps(res), file=json_out, flush=True)


if __name__ == "__main__":
    main()
