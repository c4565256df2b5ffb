"""The rocprofv3 trace summary (test1_amd/trace_summary.py) that the kernel and
host-link profiles are reduced with: its interval arithmetic against brute
force on a unit grid, and its figures on a synthetic trace whose busy times
and overlaps are known in closed form."""
import csv
import json
import random

import pytest

from test1_amd import trace_summary as ts


def _grid(spans):
    return {t for s, e in spans for t in range(s, e)}


@pytest.mark.parametrize("seed", range(20))
def test_interval_arithmetic_matches_brute_force(seed):
    rng = random.Random(seed)

    def spans(k):
        out = []
        for _ in range(k):
            s = rng.randrange(0, 60)
            out.append((s, s + rng.randrange(0, 12)))
        return out

    a, b = spans(rng.randrange(0, 8)), spans(rng.randrange(0, 8))
    ua, ub = ts.union(a), ts.union(b)
    assert ts.length(ua) == len(_grid(a))
    assert ts.inter(ua, ub) == len(_grid(a) & _grid(b))
    assert all(x[1] < y[0] for x, y in zip(ua, ua[1:]))   # disjoint, sorted, touching ones merged


def test_interval_special_cases():
    assert ts.union([(5, 7), (1, 3), (3, 5)]) == [[1, 7]]       # touching intervals merge
    assert ts.union([(0, 10), (2, 3)]) == [[0, 10]]             # nested
    assert ts.inter([[0, 10]], [[10, 20]]) == 0
    assert ts.inter([[0, 4], [6, 10]], [[2, 8]]) == 4
    assert ts.length([]) == 0 and ts.inter([], [[0, 1]]) == 0


MS = 1_000_000  # ns


def _write_trace(d, warm, steps):
    """Steps of 100 ms: lookup [0,1], casts [5,6] and [60,61], a GEMM
    [10,50], an H2D copy [40,70], a D2H copy [80,90] beside a pack kernel
    [85,95], gradient rows [98,99] (ms into the step); then 23 idle casts."""
    kernels, copies = [], []

    def k(name, s, e, grid=1):
        kernels.append({"Kernel_Name": name, "Start_Timestamp": s, "End_Timestamp": e, "Grid_Size_X": grid})

    for step in range(warm + steps):
        t = step * 100 * MS
        k("void gather_rows_kernel<true>(...)", t, t + MS)
        k("cast_flat_kernel(...)", t + 5 * MS, t + 6 * MS, 1000)
        k("Cijk_Ailk_Bljk_BBS_MT256x256x64", t + 10 * MS, t + 50 * MS)
        k("cast_flat_kernel(...)", t + 60 * MS, t + 61 * MS, 1000)
        k("void seg_kernel<OpCopy16>(...)", t + 85 * MS, t + 95 * MS)
        k("void gather_rows_kernel<false>(...)", t + 98 * MS, t + 99 * MS)
        copies.append({"Direction": "MEMORY_COPY_HOST_TO_DEVICE", "Start_Timestamp": t + 40 * MS,
                       "End_Timestamp": t + 70 * MS})
        copies.append({"Direction": "MEMORY_COPY_DEVICE_TO_HOST", "Start_Timestamp": t + 80 * MS,
                       "End_Timestamp": t + 90 * MS})
    t = (warm + steps) * 100 * MS
    for i in range(23):
        k("cast_flat_kernel(...)", t + i * MS, t + i * MS + MS // 2, 1000)
    for name, rows in (("run_kernel_trace.csv", kernels), ("run_memory_copy_trace.csv", copies)):
        with open(d / name, "w", newline="") as f:
            w = csv.DictWriter(f, fieldnames=list(rows[0]))
            w.writeheader()
            w.writerows(rows)
    with open(d / "run_kernel_stats.csv", "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=["Name", "Calls", "TotalDurationNs", "AverageNs", "Percentage"])
        w.writeheader()
        w.writerow({"Name": "cast_flat_kernel(...)", "Calls": 29, "TotalDurationNs": 17.5 * MS,
                    "AverageNs": 17.5 * MS / 29, "Percentage": 10.0})
        w.writerow({"Name": "Cijk_Ailk_Bljk_BBS_MT256x256x64", "Calls": 3, "TotalDurationNs": 120 * MS,
                    "AverageNs": 40 * MS, "Percentage": 90.0})
    bench = {"value": 1.0, "ms_per_step": 100.0,
             "roofline": {"avg_launch_ms": 1.0, "frac": 0.5, "launches": 2 * steps},
             "host_link": {"h2d": {"bytes_per_step": 3.1e9}, "d2h": {"bytes_per_step": 1.6e9}, "alone": None}}
    (d / "bench.json").write_text("[bench] log line\n" + json.dumps(bench) + "\n")


def test_summary_of_a_synthetic_trace(tmp_path, capsys):
    _write_trace(tmp_path, warm=1, steps=2)
    ts.main([str(tmp_path), "1", "2", str(tmp_path / "bench.json")])
    out = capsys.readouterr().out
    # 2 casts per step; the 4 timed ones last 1 ms and move 6 B x 8 elements x 1000 lanes
    assert "casts per step 2; timed casts 4 avg 1.0000 ms" in out
    assert "bytes/launch 48000" in out
    assert "last 20 casts (idle GPU, one layer) avg 0.5000 ms" in out
    # window: the second step's lookup (100 ms) to the third step's gradient rows (299 ms)
    assert "window 0.199 s" in out
    # H2D per step: lookup 1 ms + copy 30 ms, 10 ms of it under the GEMM; 3.1 GB x 2 steps / 62 ms
    assert "h2d: busy 0.06 s (31.2 %), 3.10 GB/step, 100.0 GB/s while busy" in out
    assert "under compute 32.3 %" in out
    # D2H per step: copy [80,90] with the pack [85,95] and the rows [98,99]: 16 ms, none under compute
    assert "d2h: busy 0.03 s (16.1 %), 1.60 GB/step, 100.0 GB/s while busy" in out
    assert "under compute 0.0 %" in out
    assert "compute (kernels but cast/pack/gather) 0.08 s (40.2 %)" in out
    assert "either direction 47.2 %, both 0.0 %" in out
    # busy per step: 1 + 1 + [10,70] 60 + [80,95] 15 + 1 = 78 ms of 100
    assert "neither copy nor kernel 21.6 %" in out
    assert "H2D copies longer than 8 ms: 2, durations median 30.0 ms" in out


def test_forward_and_backward_casts_of_a_kernel_only_trace(tmp_path, capsys):
    """Casts after each step's largest (the output unit's) are the
    backward's; without a memory-copy trace the host-link part is skipped."""
    kernels = []

    def k(name, s, e, grid):
        kernels.append({"Kernel_Name": name, "Start_Timestamp": s, "End_Timestamp": e, "Grid_Size_X": grid})

    for step in range(3):   # 1 warmup + 2 timed steps of 100 ms
        t = step * 100 * MS
        k("cast_flat_kernel(...)", t, t + MS, 10**8)                      # a decoder, forward
        k("cast_flat_kernel(...)", t + 10 * MS, t + 13 * MS, 3 * 10**8)   # the output unit
        k("Cijk_Ailk_Bljk_BBS_MT256x256x64", t + 20 * MS, t + 50 * MS, 1)
        k("cast_flat_kernel(...)", t + 60 * MS, t + 62 * MS, 10**8)       # a decoder's reload
    for i in range(23):
        k("cast_flat_kernel(...)", 400 * MS + i * MS, 400 * MS + i * MS + MS // 2, 10**8)
    with open(tmp_path / "run_kernel_trace.csv", "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=list(kernels[0]))
        w.writeheader()
        w.writerows(kernels)
    with open(tmp_path / "run_kernel_stats.csv", "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=["Name", "Calls", "TotalDurationNs", "AverageNs", "Percentage"])
        w.writeheader()
        w.writerow({"Name": "cast_flat_kernel(...)", "Calls": 32, "TotalDurationNs": 30 * MS,
                    "AverageNs": 30 * MS / 32, "Percentage": 25.0})
    bench = {"value": 1.0, "ms_per_step": 100.0, "roofline": {"avg_launch_ms": 2.0, "frac": 0.5, "launches": 6}}
    (tmp_path / "bench.json").write_text(json.dumps(bench) + "\n")
    ts.main([str(tmp_path), "1", "2", str(tmp_path / "bench.json")])
    out = capsys.readouterr().out
    assert "casts per step 3; timed casts 6 avg 2.0000 ms" in out
    # forward: 1 and 3 ms for 4.8 and 14.4 GB; backward: 2 ms for 4.8 GB
    assert "forward: 4 casts avg 2.0000 ms, 0.6000 of 8 TB/s" in out
    assert "backward: 2 casts avg 2.0000 ms, 0.3000 of 8 TB/s" in out
    assert "window" not in out and "h2d:" not in out
