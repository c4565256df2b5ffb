"""Summary of a rocprofv3 kernel and memory-copy trace of one ``bench.py`` run.

    python -m test1_amd.trace_summary DIR WARMUP STEPS BENCH_JSON

DIR holds the run's ``run_kernel_trace.csv``, ``run_kernel_stats.csv`` and
``run_memory_copy_trace.csv`` (``rocprofv3 --kernel-trace --memory-copy-trace
--stats --output-format csv -d DIR -o run -- python3 bench.py ...``);
BENCH_JSON is the JSON line the same run printed (its bytes per step and
figures).  Prints:
  - the staging cast over the timed steps (the dispatches after the warmup
    steps' and before the bench's 23 idle-GPU launches): average duration and
    rate against 8 TB/s, next to the bench's own event-timed figure, and
    split into the forward's casts and the backward's (those after each
    step's largest cast, the output unit's);
  - the ten kernels with the most time;
  - the host link over the timed steps, from the first timed step's embedding
    lookup to the last one's gradient rows: each direction's busy time (union
    of the DMA copies and the host-link kernels: lookup and checkpoint pack /
    gradient rows), its rate while busy from the bench's bytes per step, and
    the share of it under other kernels (skipped for a trace without
    ``run_memory_copy_trace.csv``).
"""
import csv
import json
import os
import statistics
import sys


def union(spans):
    """Merged, sorted ``[start, end]`` intervals covering ``spans``."""
    out = []
    for s, e in sorted(tuple(x) for x in spans):
        if out and s <= out[-1][1]:
            out[-1][1] = max(out[-1][1], e)
        else:
            out.append([s, e])
    return out


def length(u) -> int:
    """Total length of disjoint intervals."""
    return sum(e - s for s, e in u)


def inter(a, b) -> int:
    """Length of the intersection of two sorted lists of disjoint intervals."""
    i = j = 0
    tot = 0
    while i < len(a) and j < len(b):
        lo, hi = max(a[i][0], b[j][0]), min(a[i][1], b[j][1])
        if hi > lo:
            tot += hi - lo
        if a[i][1] < b[j][1]:
            i += 1
        else:
            j += 1
    return tot


def main(argv=None) -> None:
    d, warm, steps, bj = (sys.argv[1:] if argv is None else argv)[:4]
    warm, steps = int(warm), int(steps)
    B = json.loads([ln for ln in open(bj) if ln.startswith("{")][-1])
    rows = sorted(csv.DictReader(open(f"{d}/run_kernel_trace.csv")), key=lambda r: int(r["Start_Timestamp"]))
    iv = lambda r: (int(r["Start_Timestamp"]), int(r["End_Timestamp"]))
    cast = [r for r in rows if "cast_flat_kernel" in r["Kernel_Name"]]
    n_step = (len(cast) - 23) // (warm + steps)
    timed = cast[n_step * warm:n_step * (warm + steps)]
    dur = [(int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e6 for r in timed]
    elems = [int(r["Grid_Size_X"]) * 8 for r in timed]
    avg = sum(dur) / len(dur)
    ab = 6 * sum(elems) / len(elems)
    print(f"bench: {B['value']:.0f} tokens/s, {B['ms_per_step']:.1f} ms/step; bench cast avg {B['roofline']['avg_launch_ms']:.4f} ms frac {B['roofline']['frac']:.4f} ({B['roofline']['launches']} launches)")
    print(f"casts per step {n_step}; timed casts {len(timed)} avg {avg:.4f} ms median {statistics.median(dur):.4f} ms; "
          f"bytes/launch {ab:.0f}; {ab / avg / 1e6:.1f} GB/s = {ab / avg / 1e6 / 8000:.4f} of 8 TB/s")
    # Each step's casts after its largest one (the output unit's, the last
    # of the forward) are the backward's reloads (fp32 reloads only).
    for what, pick in (("forward", lambda st, big: st[:big + 1]), ("backward", lambda st, big: st[big + 1:])):
        part = []
        for k in range(steps):
            st = timed[k * n_step:(k + 1) * n_step]
            big = max(range(len(st)), key=lambda i: int(st[i]["Grid_Size_X"]))
            part += pick(st, big)
        if part:
            pd = sum((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e6 for r in part) / len(part)
            pb = 6 * 8 * sum(int(r["Grid_Size_X"]) for r in part) / len(part)
            print(f"  {what}: {len(part)} casts avg {pd:.4f} ms, {pb / pd / 1e6 / 8000:.4f} of 8 TB/s")
    alone = cast[-20:]
    ad = [(int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e6 for r in alone]
    print(f"last 20 casts (idle GPU, one layer) avg {sum(ad) / len(ad):.4f} ms")
    for r in csv.DictReader(open(f"{d}/run_kernel_stats.csv")):
        if "cast_flat_kernel" in r["Name"]:
            print(f"stats: cast calls {r['Calls']} avg {float(r['AverageNs']) / 1e6:.4f} ms")
    st = sorted(csv.DictReader(open(f"{d}/run_kernel_stats.csv")), key=lambda r: -float(r["TotalDurationNs"]))
    print("top kernels (whole run): name | calls | total ms | avg us | %")
    for r in st[:10]:
        print(f"  {r['Name'][:70]} | {r['Calls']} | {float(r['TotalDurationNs']) / 1e6:.1f} | {float(r['AverageNs']) / 1e3:.1f} | {r['Percentage']}")
    # host link over the timed steps (needs the memory-copy trace)
    if not os.path.exists(f"{d}/run_memory_copy_trace.csv"):
        return
    C = list(csv.DictReader(open(f"{d}/run_memory_copy_trace.csv")))
    look = sorted(iv(r) for r in rows if "gather_rows_kernel<true" in r["Kernel_Name"])
    grow = sorted(iv(r) for r in rows if "gather_rows_kernel<false" in r["Kernel_Name"])
    w0, w1 = look[warm][0], grow[warm + steps - 1][1]

    def clip(sp):
        return [(max(s, w0), min(e, w1)) for s, e in sp if e > w0 and s < w1]

    h2d = union(clip([iv(r) for r in C if r["Direction"].endswith("HOST_TO_DEVICE")] + look))
    d2h = union(clip([iv(r) for r in C if r["Direction"].endswith("DEVICE_TO_HOST")] + grow +
                     [iv(r) for r in rows if "seg_kernel" in r["Kernel_Name"]]))
    comp = union(clip([iv(r) for r in rows if not any(x in r["Kernel_Name"] for x in ("cast_flat", "seg_kernel", "gather_rows"))]))
    W = w1 - w0
    hl = B["host_link"]
    hb = hl["h2d"]["bytes_per_step"]
    db = hl["d2h"]["bytes_per_step"] + hl["d2h"].get("untimed_bytes_per_step", 0.0)
    print(f"window {W / 1e9:.3f} s, {W / 1e6 / steps:.1f} ms/step (first timed lookup to last timed gradient rows)")
    for name, u, b in (("h2d", h2d, hb), ("d2h", d2h, db)):
        L = length(u)
        print(f"{name}: busy {L / 1e9:.2f} s ({100 * L / W:.1f} %), {b / 1e9:.2f} GB/step, {b * steps / L:.1f} GB/s while busy "
              f"({b * steps / L / 63:.3f} of 63), under compute {100 * inter(u, comp) / L:.1f} %")
    print(f"compute (kernels but cast/pack/gather) {length(comp) / 1e9:.2f} s ({100 * length(comp) / W:.1f} %)")
    print(f"either direction {100 * length(union(h2d + d2h)) / W:.1f} %, both {100 * inter(h2d, d2h) / W:.1f} %")
    allu = union(h2d + d2h + comp + clip([iv(r) for r in rows]))
    print(f"neither copy nor kernel {100 * (W - length(allu)) / W:.1f} %")
    big = [x for x in clip([iv(r) for r in C if r["Direction"].endswith("HOST_TO_DEVICE")]) if x[1] - x[0] > 8e6]
    rates = sorted((e - s) / 1e6 for s, e in big)
    print(f"H2D copies longer than 8 ms: {len(big)}, durations median {statistics.median(rates):.1f} ms, max {rates[-1]:.1f} ms")
    print("alone:", hl.get("alone"))


if __name__ == "__main__":
    main()
