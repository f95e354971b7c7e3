"""Per-kernel summary of rocprofv3 CSV output (kernel traces and counter collections) for the
`kernels.bench.profile_cases` workload: one row per (kernel, grid size) with the median duration,
HBM bytes from FETCH_SIZE / WRITE_SIZE scaled by the calibration pass the workload runs first
(torch.neg over 64 MiB of fp16: exactly 65536 KiB read and written per dispatch), VALUBusy and
MfmaUtil.

    python3 -m kernels.bench.counters DIR [DIR ...] [--md out.md]

DIR holds any of `*_kernel_trace.csv` and `*_counter_collection.csv` (one rocprofv3 run each).
"""

from __future__ import annotations

import argparse
import csv
import re
import statistics
import sys
from collections import defaultdict
from pathlib import Path

COPY_KIB = 65536.0


def short_name(name: str) -> str:
    """`void (anonymous namespace)::w4a16_m1_kernel<8, 6, 4, 0>(...)` -> `w4a16_m1_kernel<8, 6, 4, 0>`."""
    n = name.strip().strip('"')
    n = re.sub(r"^void ", "", n)
    n = re.sub(r"\(anonymous namespace\)::", "", n)
    depth, out = 0, []
    for ch in n:  # drop the argument list (the first '(' outside template brackets)
        if ch == "<":
            depth += 1
        elif ch == ">":
            depth -= 1
        elif ch == "(" and depth == 0:
            break
        out.append(ch)
    return "".join(out)[:90]


def _grid(row: dict) -> int:
    if row.get("Grid_Size"):
        return int(float(row["Grid_Size"]))
    g = 1
    for k in ("Grid_Size_X", "Grid_Size_Y", "Grid_Size_Z"):
        if row.get(k):
            g *= int(float(row[k]))
    return g


def load(dirs):
    durations = defaultdict(list)            # (kernel, grid) -> [ns]
    counters = defaultdict(lambda: defaultdict(list))  # (kernel, grid) -> counter -> [values]
    order = {}
    for d in dirs:
        for path in sorted(Path(d).rglob("*_kernel_trace.csv")):
            with open(path) as f:
                for row in csv.DictReader(f):
                    key = (short_name(row["Kernel_Name"]), _grid(row))
                    durations[key].append(int(row["End_Timestamp"]) - int(row["Start_Timestamp"]))
                    order.setdefault(key, int(row.get("Dispatch_Id", len(order))))
        for path in sorted(Path(d).rglob("*_counter_collection.csv")):
            per_dispatch = defaultdict(float)
            keys = {}
            with open(path) as f:
                for row in csv.DictReader(f):
                    key = (short_name(row["Kernel_Name"]), _grid(row))
                    did = row.get("Dispatch_Id") or row.get("Correlation_Id")
                    per_dispatch[(key, did, row["Counter_Name"])] += float(row["Counter_Value"])
                    keys[key] = True
                    order.setdefault(key, int(did) if did and did.isdigit() else len(order))
            for (key, _did, cname), v in per_dispatch.items():
                counters[key][cname].append(v)
    return durations, counters, order


def summarize(durations, counters, order):
    med = statistics.median
    fetch_f = write_f = None
    for (name, _grid), cs in counters.items():
        if "neg_kernel" in name:
            if cs.get("FETCH_SIZE"):
                fetch_f = COPY_KIB / med(cs["FETCH_SIZE"])
            if cs.get("WRITE_SIZE"):
                write_f = COPY_KIB / med(cs["WRITE_SIZE"])
    rows = []
    for key in sorted(set(durations) | set(counters), key=lambda k: order.get(k, 0)):
        cs = counters.get(key, {})
        r = {"kernel": key[0], "grid": key[1], "dispatches": len(durations.get(key, [])) or None,
             "median_ns": med(durations[key]) if durations.get(key) else None}
        if cs.get("FETCH_SIZE"):
            r["fetch_kib"] = med(cs["FETCH_SIZE"])
            r["read_bytes"] = r["fetch_kib"] * 1024 * fetch_f if fetch_f else None
        if cs.get("WRITE_SIZE"):
            r["write_kib"] = med(cs["WRITE_SIZE"])
            r["write_bytes"] = r["write_kib"] * 1024 * write_f if write_f else None
        for c in ("VALUBusy", "MfmaUtil"):
            if cs.get(c):
                r[c] = med(cs[c])
        rows.append(r)
    return rows, fetch_f, write_f


def markdown(rows, fetch_f, write_f) -> str:
    def f(v, fmt):
        return "—" if v is None else format(v, fmt)

    out = [f"FETCH_SIZE scale {f(fetch_f, '.4f')}, WRITE_SIZE scale {f(write_f, '.4f')} "
           "(torch.neg over 64 MiB: 65536 KiB read and written per dispatch)", "",
           "| kernel | grid | dispatches | median µs | HBM read B | HBM write B | VALUBusy % | MfmaUtil % |",
           "|---|---|---|---|---|---|---|---|"]
    for r in rows:
        us = None if r.get("median_ns") is None else r["median_ns"] / 1e3
        out.append(f"| `{r['kernel']}` | {r['grid']} | {r.get('dispatches') or '—'} | {f(us, '.2f')} | "
                   f"{f(r.get('read_bytes'), ',.0f')} | {f(r.get('write_bytes'), ',.0f')} | "
                   f"{f(r.get('VALUBusy'), '.1f')} | {f(r.get('MfmaUtil'), '.1f')} |")
    return "\n".join(out) + "\n"


def main(argv=None) -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("dirs", nargs="+")
    ap.add_argument("--md", default=None)
    args = ap.parse_args(argv)
    rows, ff, wf = summarize(*load(args.dirs))
    text = markdown(rows, ff, wf)
    if args.md:
        Path(args.md).write_text(text)
    sys.stdout.write(text)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
