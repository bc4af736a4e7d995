"""Summaries of rocprofv3 CSV output (kernel-trace stats and PMC counters).

Usage, after ``rocprofv3 ... --output-format csv -d DIR -o NAME -- <program>``:

    python -m gmdn_amd.profiling stats DIR [--kernel REGEX]  # per-kernel durations
    python -m gmdn_amd.profiling traffic --kernel REGEX \\
        --fetch DIR1 --write DIR2 --copy-fetch DIR3 --copy-write DIR4 \\
        --copy-bytes N

``traffic`` turns the FETCH_SIZE / WRITE_SIZE derived counters (KiB per
dispatch) into HBM bytes per launch of the kernels matching REGEX (summed
over the kernels when the op runs several).  Each
counter is scaled by what it reads for a plain device copy of N bytes
(N read + N written), so the figure is in the same units as the algorithmic
bytes.  The output is markdown; its ``traffic_bytes_per_launch:`` line is
what bench.py reads back.
"""
from __future__ import annotations

import argparse
import csv
import glob
import os
import re
import statistics


def _find(d: str, suffix: str) -> str:
    hits = sorted(glob.glob(os.path.join(d, "**", f"*{suffix}"), recursive=True))
    if not hits:
        raise FileNotFoundError(f"no *{suffix} under {d}")
    return hits[0]


def kernel_stats(d: str):
    """Rows of ``*_kernel_stats.csv``: (name, calls, avg_ns, min_ns, max_ns, pct)."""
    rows = []
    with open(_find(d, "kernel_stats.csv")) as f:
        for r in csv.DictReader(f):
            rows.append((r["Name"], int(r["Calls"]), float(r["AverageNs"]), float(r["MinNs"]),
                         float(r["MaxNs"]), float(r["Percentage"])))
    rows.sort(key=lambda r: -r[1] * r[2])
    return rows


def counter_per_dispatch(d: str, counter: str, kernel_regex: str):
    """Per-dispatch values of ``counter`` for kernels whose name matches the regex."""
    pat = re.compile(kernel_regex)
    vals = {}
    with open(_find(d, "counter_collection.csv")) as f:
        for r in csv.DictReader(f):
            if r["Counter_Name"] != counter or not pat.search(r["Kernel_Name"]):
                continue
            key = r["Dispatch_Id"]
            vals[key] = vals.get(key, 0.0) + float(r["Counter_Value"])
    if not vals:
        raise ValueError(f"no {counter} rows for /{kernel_regex}/ under {d}")
    return list(vals.values())


def counter_by_kernel(d: str, counter: str, kernel_regex: str):
    """{kernel name: per-dispatch values of ``counter``} for matching kernels."""
    pat = re.compile(kernel_regex)
    per = {}
    with open(_find(d, "counter_collection.csv")) as f:
        for r in csv.DictReader(f):
            if r["Counter_Name"] != counter or not pat.search(r["Kernel_Name"]):
                continue
            k = (r["Kernel_Name"], r["Dispatch_Id"])
            per[k] = per.get(k, 0.0) + float(r["Counter_Value"])
    out = {}
    for (name, _), v in per.items():
        out.setdefault(name, []).append(v)
    if not out:
        raise ValueError(f"no {counter} rows for /{kernel_regex}/ under {d}")
    return out


def _per_launch(d: str, counter: str, kernel_regex: str) -> float:
    """Sum over the matching kernels of each one's median per-dispatch value:
    the counter for one launch of the op when it runs those kernels once each."""
    return sum(statistics.median(v) for v in counter_by_kernel(d, counter, kernel_regex).values())


def _stats_md(d: str, kernel_regex: str = "") -> str:
    out = ["| kernel | calls | avg us | min us | max us | % time |", "|---|---|---|---|---|---|"]
    pat = re.compile(kernel_regex)
    for name, calls, avg, mn, mx, pct in kernel_stats(d):
        if not pat.search(name):
            continue
        out.append(f"| `{name}` | {calls} | {avg / 1e3:.1f} | {mn / 1e3:.1f} | {mx / 1e3:.1f} | {pct:.1f} |")
    return "\n".join(out)


def _traffic_md(a) -> str:
    kib = 1024.0
    fetch = _per_launch(a.fetch, "FETCH_SIZE", a.kernel)
    write = _per_launch(a.write, "WRITE_SIZE", a.kernel)
    cf = statistics.median(counter_per_dispatch(a.copy_fetch, "FETCH_SIZE", a.copy_kernel))
    cw = statistics.median(counter_per_dispatch(a.copy_write, "WRITE_SIZE", a.copy_kernel))
    sf, sw = a.copy_bytes / (cf * kib), a.copy_bytes / (cw * kib)
    rd, wr = fetch * kib * sf, write * kib * sw
    return "\n".join([
        f"kernel /{a.kernel}/, copy kernel /{a.copy_kernel}/ over {a.copy_bytes} bytes", "",
        "| counter | kernel KiB/dispatch | copy KiB/dispatch | scale (copy bytes / counter bytes) | kernel bytes |",
        "|---|---|---|---|---|",
        f"| FETCH_SIZE | {fetch:.1f} | {cf:.1f} | {sf:.4f} | {rd:.0f} |",
        f"| WRITE_SIZE | {write:.1f} | {cw:.1f} | {sw:.4f} | {wr:.0f} |", "",
        f"traffic_bytes_per_launch: {rd + wr:.0f}",
        f"read_bytes_per_launch: {rd:.0f}",
        f"write_bytes_per_launch: {wr:.0f}",
    ])


def read_traffic(path: str):
    """The ``traffic_bytes_per_launch`` figure of a summary written by ``traffic``, or None."""
    if not os.path.exists(path):
        return None
    with open(path) as f:
        for line in f:
            if line.startswith("traffic_bytes_per_launch:"):
                return float(line.split(":", 1)[1])
    return None


def main(argv=None):
    p = argparse.ArgumentParser(prog="python -m gmdn_amd.profiling")
    sub = p.add_subparsers(dest="cmd", required=True)
    s = sub.add_parser("stats")
    s.add_argument("dir")
    s.add_argument("--kernel", default="", help="only kernels whose name matches this regex")
    t = sub.add_parser("traffic")
    t.add_argument("--kernel", required=True)
    t.add_argument("--copy-kernel", default="copy|elementwise")
    t.add_argument("--fetch", required=True)
    t.add_argument("--write", required=True)
    t.add_argument("--copy-fetch", required=True)
    t.add_argument("--copy-write", required=True)
    t.add_argument("--copy-bytes", type=int, required=True)
    a = p.parse_args(argv)
    print(_stats_md(a.dir, a.kernel) if a.cmd == "stats" else _traffic_md(a))


if __name__ == "__main__":
    main()
