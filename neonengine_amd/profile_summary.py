"""Summarise rocprofv3 output of the decode loop.

    python -m neonengine_amd.profile_summary <run_kernel_trace.csv> \
        --last-steps K --kernels-per-step N [--bytes name=BYTES ...]
    python -m neonengine_amd.profile_summary --pmc <run_counter_collection.csv>
    python -m neonengine_amd.profile_summary --segments <run_kernel_trace.csv>

The first form reads a kernel trace; the second averages each counter per
dispatch and kernel name (rocprofv3 --pmc output, e.g. FETCH_SIZE and
WRITE_SIZE in KiB per dispatch); the third splits a trace into segments of
consecutive dispatches of one kernel with one grid, or of two kernels in
turn (a sweep point's timed launches), and prints each segment's count and
average duration in order.

Keeps the last K decode steps (K * N dispatches; the gpt-oss step has
N = 1 + 6 n_layers + (one attention merge per layer with several key splits)
+ 2, i.e. 159 at the 20b shape with a 4096-row cache), groups the dispatches
by kernel name and prints a Markdown
table: calls per step, average duration, share of step time, and -- for the
kernels given algorithmic bytes per launch -- achieved GB/s.
"""
from __future__ import annotations

import argparse
import csv
import re
import sys
from collections import defaultdict


def short(name: str) -> str:
    name = re.sub(r"\(.*$", "", name)          # drop argument list
    name = re.sub(r"^void\s+", "", name)
    name = name.replace("neon::", "")
    return name


def pmc_summary(path: str):
    vals = defaultdict(float)
    disp = defaultdict(set)
    with open(path) as f:
        for r in csv.DictReader(f):
            key = (short(r["Kernel_Name"]), r["Counter_Name"])
            vals[key] += float(r["Counter_Value"])
            disp[key].add(r.get("Dispatch_Id") or r.get("Correlation_Id"))
    print("| kernel | counter | dispatches | avg per dispatch |")
    print("|---|---|---|---|")
    for key in sorted(vals):
        n = len(disp[key])
        print(f"| {key[0]} | {key[1]} | {n} | {vals[key] / n:.1f} |")


def segments(path: str, min_count: int):
    """Runs of consecutive dispatches that repeat one kernel (one grid), or a
    pair of kernels in turn (a split kernel and its merge): one row per run,
    with the average duration of one repetition (the pair's sum)."""
    rows = []
    with open(path) as f:
        for r in csv.DictReader(f):
            grid = tuple(r.get(f"Grid_Size_{d}", "") for d in "XYZ")
            rows.append((int(r["Start_Timestamp"]), int(r["End_Timestamp"]),
                         (short(r["Kernel_Name"]), "x".join(grid))))
    rows.sort()
    rows = [r for r in rows if not r[2][0].startswith("__amd")]
    segs, i = [], 0
    while i < len(rows):
        key = rows[i][2]
        period = 1
        if (i + 2 < len(rows) and rows[i + 1][2] != key and rows[i + 2][2] == key
                and (i + 3 >= len(rows) or rows[i + 3][2] == rows[i + 1][2])):
            period = 2
        unit = [rows[i + j][2] for j in range(period)]
        reps = []
        while i + period <= len(rows) and [rows[i + j][2] for j in range(period)] == unit:
            reps.append(sum(rows[i + j][1] - rows[i + j][0] for j in range(period)))
            i += period
        segs.append((unit, reps))
    print("| segment | kernel(s) | grid(s) | repetitions | avg us | min us |")
    print("|---|---|---|---|---|---|")
    n = 0
    for unit, d in segs:
        if len(d) < min_count:
            continue
        print(f"| {n} | {' + '.join(k for k, _ in unit)} | {' + '.join(g for _, g in unit)} | "
              f"{len(d)} | {sum(d) / len(d) / 1e3:.2f} | {min(d) / 1e3:.2f} |")
        n += 1


def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("trace")
    ap.add_argument("--pmc", action="store_true", help="the file is counter_collection.csv")
    ap.add_argument("--segments", action="store_true",
                    help="per-segment table of consecutive same-kernel, same-grid dispatches")
    ap.add_argument("--min-count", type=int, default=8,
                    help="--segments: skip segments with fewer dispatches")
    ap.add_argument("--last-steps", type=int)
    ap.add_argument("--kernels-per-step", type=int)
    ap.add_argument("--bytes", action="append", default=[],
                    help="kernel-name-regex=bytes_per_launch")
    ap.add_argument("--layer-parity", action="store_true",
                    help="also split per-layer kernels by layer parity (even layers are "
                         "the sliding-window layers of gpt-oss)")
    a = ap.parse_args(argv)
    if a.pmc:
        pmc_summary(a.trace)
        return
    if a.segments:
        segments(a.trace, a.min_count)
        return
    if not a.last_steps or not a.kernels_per_step:
        sys.exit("--last-steps and --kernels-per-step are required for a kernel trace")
    rows = []
    with open(a.trace) as f:
        for r in csv.DictReader(f):
            rows.append((int(r["Start_Timestamp"]), int(r["End_Timestamp"]), r["Kernel_Name"]))
    rows.sort()
    # runtime copy kernels (reads of results) are not part of a step
    rows = [r for r in rows if not short(r[2]).startswith("__amd")]
    n = a.last_steps * a.kernels_per_step
    if len(rows) < n:
        sys.exit(f"trace has {len(rows)} dispatches, fewer than {n}")
    rows = rows[-n:]
    span_ns = rows[-1][1] - rows[0][0]
    busy = defaultdict(int)
    cnt = defaultdict(int)
    for s, e, k in rows:
        busy[short(k)] += e - s
        cnt[short(k)] += 1
    total_busy = sum(busy.values())
    byts = {}
    for spec in a.bytes:
        pat, b = spec.rsplit("=", 1)
        byts[pat] = int(b)
    step_us = span_ns / a.last_steps / 1e3
    print(f"decode steps: {a.last_steps}; wall per step {step_us:.1f} us; "
          f"kernel-busy per step {total_busy / a.last_steps / 1e3:.1f} us "
          f"({100 * total_busy / span_ns:.1f}% of wall; the rest is launch gaps)\n")
    print("| kernel | calls/step | avg us | us/step | % busy | GB/s |")
    print("|---|---|---|---|---|---|")
    for k in sorted(busy, key=lambda k: -busy[k]):
        avg = busy[k] / cnt[k] / 1e3
        gbs = ""
        for pat, b in byts.items():
            if re.search(pat, k):
                gbs = f"{b / (avg * 1e-6) / 1e9:.0f}"
        print(f"| {k} | {cnt[k] / a.last_steps:g} | {avg:.2f} | "
              f"{busy[k] / a.last_steps / 1e3:.1f} | {100 * busy[k] / total_busy:.1f} | {gbs} |")
    if a.layer_parity:
        # occurrence index of each kernel inside its step: for a kernel launched
        # once per layer, even occurrences are even layers
        par = defaultdict(list)
        for st in range(a.last_steps):
            seen = defaultdict(int)
            for s, e, k in rows[st * a.kernels_per_step:(st + 1) * a.kernels_per_step]:
                name = short(k)
                par[(name, seen[name] % 2)].append(e - s)
                seen[name] += 1
        print("\n| kernel | even occurrences avg us | odd occurrences avg us |")
        print("|---|---|---|")
        for k in sorted(busy, key=lambda k: -busy[k]):
            ev, od = par.get((k, 0), []), par.get((k, 1), [])
            if not od:
                continue
            print(f"| {k} | {sum(ev) / len(ev) / 1e3:.2f} | {sum(od) / len(od) / 1e3:.2f} |")


if __name__ == "__main__":
    main()
