"""Kernel-trace summaries for the measurement notes.

Reads the ``<prefix>_kernel_trace.csv`` that ``rocprofv3 --kernel-trace
--output-format csv`` writes and prints, per kernel, the dispatch count and
the mean / median / min / max duration.  With ``--tail-ops N --op-kernels
A,B`` it also summarises the last N ops of the run, where an op is one
dispatch of each named kernel in order (the GQA decode op is the split-K
kernel then the merge kernel): the mean duration of each kernel over those
ops, their sum, and the span from the first op's start to the last op's end
divided by N.  ``bench.py``'s stack workload ends with a replay of a graph of
10 x K GQA decode ops, so ``--tail-ops 10K`` selects exactly the launches
whose event time the bench line's roofline reports.

    python -m ds4f_hip.trace gpurun_out/prof/run_kernel_trace.csv \\
        --tail-ops 200 --op-kernels gqa_split_kernel,gqa_merge_kernel
"""
from __future__ import annotations

import argparse
import csv
import json
import statistics
import sys


def load(path: str):
    """Dispatches in start order: (kernel name, start ns, end ns)."""
    rows = []
    with open(path) as f:
        for r in csv.DictReader(f):
            rows.append((r["Kernel_Name"], int(r["Start_Timestamp"]), int(r["End_Timestamp"])))
    rows.sort(key=lambda x: x[1])
    return rows


def short(name: str) -> str:
    """The kernel's own name, without return type, namespaces and parameter
    list (a template argument list is kept: gqa_merge_kernel<2>)."""
    n = name.replace("(anonymous namespace)::", "")
    if n.startswith("void "):
        n = n[5:]
    n = n.split("(")[0]
    return n.split("::")[-1]


def per_kernel(rows):
    """{short name: [durations in us]}"""
    out: dict[str, list[float]] = {}
    for name, t0, t1 in rows:
        out.setdefault(short(name), []).append((t1 - t0) / 1e3)
    return out


def tail_ops(rows, n_ops: int, kernels: list[str]):
    """The last n_ops ops, an op being one dispatch of each kernel of
    `kernels` in order; returns per-kernel duration lists and the span (us)."""
    sel = [r for r in rows if any(short(r[0]).startswith(k) for k in kernels)]
    need = n_ops * len(kernels)
    if len(sel) < need:
        raise SystemExit(f"only {len(sel)} dispatches of {kernels}, {need} needed")
    sel = sel[-need:]
    for i, r in enumerate(sel):
        want = kernels[i % len(kernels)]
        if not short(r[0]).startswith(want):
            raise SystemExit(f"dispatch {i} of the tail is {short(r[0])}, expected {want}")
    durs = {k: [(r[2] - r[1]) / 1e3 for i, r in enumerate(sel) if i % len(kernels) == j]
            for j, k in enumerate(kernels)}
    span = (sel[-1][2] - sel[0][1]) / 1e3
    return durs, span


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("csv")
    ap.add_argument("--tail-ops", type=int, default=0)
    ap.add_argument("--op-kernels", default="gqa_split_kernel,gqa_merge_kernel")
    ap.add_argument("--json", action="store_true", help="one JSON object instead of tables")
    a = ap.parse_args(argv)
    rows = load(a.csv)
    res = {"kernels": {}}
    for k, d in sorted(per_kernel(rows).items(), key=lambda kv: -sum(kv[1])):
        res["kernels"][k] = {"dispatches": len(d), "mean_us": statistics.fmean(d),
                             "median_us": statistics.median(d), "min_us": min(d), "max_us": max(d)}
    if a.tail_ops:
        ks = a.op_kernels.split(",")
        durs, span = tail_ops(rows, a.tail_ops, ks)
        res["tail"] = {"ops": a.tail_ops, "kernels": ks,
                       "mean_us": {k: statistics.fmean(v) for k, v in durs.items()},
                       "sum_of_means_us": sum(statistics.fmean(v) for v in durs.values()),
                       "span_per_op_us": span / a.tail_ops}
    if a.json:
        print(json.dumps(res))
        return 0
    print("| kernel | dispatches | mean us | median us | min us | max us |")
    print("|---|---|---|---|---|---|")
    for k, s in res["kernels"].items():
        print(f"| {k} | {s['dispatches']} | {s['mean_us']:.3f} | {s['median_us']:.3f} | "
              f"{s['min_us']:.3f} | {s['max_us']:.3f} |")
    if a.tail_ops:
        t = res["tail"]
        print()
        print(f"last {t['ops']} ops of {' + '.join(t['kernels'])}: " +
              ", ".join(f"{k} {v:.3f} us" for k, v in t["mean_us"].items()) +
              f"; sum {t['sum_of_means_us']:.3f} us; span per op {t['span_per_op_us']:.3f} us")
    return 0


if __name__ == "__main__":
    sys.exit(main())
