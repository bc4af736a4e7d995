"""Summaries of rocprofv3 CSV output (kernel-trace stats and PMC counters).

Usage, after ``rocprofv3 ... --output-format csv -d DIR -o NAME -- <program>``:

    python -m gmdn_amd.profiling stats DIR [--kernel REGEX]  # per-kernel durations
    python -m gmdn_amd.profiling traffic --kernel REGEX \\
        --fetch DIR1 --write DIR2 --copy-fetch DIR3 --copy-write DIR4 \\
        --copy-bytes N

    python -m gmdn_amd.profiling mfma DIR [--kernel REGEX] [--simds 1024]

``mfma`` reads one PMC pass of SQ_INSTS_VALU_MFMA_MOPS_BF16 (and, when
collected, SQ_INSTS_VALU_MFMA_MOPS_F32), SQ_VALU_MFMA_BUSY_CYCLES and
GRBM_GUI_ACTIVE and gives per kernel (medians over its dispatches): the bf16
MFMA flops issued (MOPS x 512), their rate over the dispatch's own duration,
that rate as a fraction of the 2.5 PFLOP/s dense bf16 peak, the fp32 MFMA
flops and their fraction of the 157.3 TFLOP/s fp32 peak, and MfmaUtil =
busy cycles / (one XCD's GUI-active cycles x SIMDs), rocprofv3's own
definition.

``traffic`` turns the FETCH_SIZE / WRITE_SIZE derived counters (KiB per
dispatch) into HBM bytes per launch of the kernels matching REGEX (summed
over the kernels when the op runs several).  Each
counter is scaled by what it reads for a plain device copy of N bytes
(N read + N written), so the figure is in the same units as the algorithmic
bytes.  ``--calls-per-op K`` sums K dispatches of each kernel per launch (their
mean times K) for an op that runs its kernels in K segments.  The output is markdown; its ``traffic_bytes_per_launch:`` line is
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


def _per_launch(d: str, counter: str, kernel_regex: str, calls_per_op: int = 1) -> float:
    """The counter for one launch of the op: with calls_per_op = 1 (the op
    runs each matching kernel once) the sum over the kernels of each one's
    median per-dispatch value; otherwise each kernel's mean per dispatch times
    calls_per_op (an op that runs every kernel that many times, in dispatches
    of different sizes, such as a scan in chunk segments)."""
    per = counter_by_kernel(d, counter, kernel_regex).values()
    if calls_per_op == 1:
        return sum(statistics.median(v) for v in per)
    return sum(statistics.fmean(v) * calls_per_op for v in per)


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
    fetch = _per_launch(a.fetch, "FETCH_SIZE", a.kernel, a.calls_per_op)
    write = _per_launch(a.write, "WRITE_SIZE", a.kernel, a.calls_per_op)
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


BF16_PEAK_TFLOPS = 2500.0
F32_PEAK_TFLOPS = 157.3


def mfma_by_kernel(d: str, kernel_regex: str = "", simds: int = 1024, xcds: int = 8):
    """{kernel: dict(dispatches, flops, us, tflops, frac, util)} from one PMC
    pass of the three MFMA counters (medians over the kernel's dispatches).
    rocprofv3 reports GRBM_GUI_ACTIVE summed over the XCDs; MfmaUtil takes
    one XCD's count (its expression reduces the counter with max)."""
    pat = re.compile(kernel_regex)
    disp = {}
    with open(_find(d, "counter_collection.csv")) as f:
        for r in csv.DictReader(f):
            if not pat.search(r["Kernel_Name"]):
                continue
            key = (r["Kernel_Name"], r["Dispatch_Id"])
            e = disp.setdefault(key, {"ns": int(r["End_Timestamp"]) - int(r["Start_Timestamp"])})
            e[r["Counter_Name"]] = e.get(r["Counter_Name"], 0.0) + float(r["Counter_Value"])
    per = {}
    for (name, _), e in disp.items():
        per.setdefault(name, []).append(e)
    out = {}
    for name, es in per.items():
        flops = statistics.median(e.get("SQ_INSTS_VALU_MFMA_MOPS_BF16", 0.0) * 512 for e in es)
        f32 = statistics.median(e.get("SQ_INSTS_VALU_MFMA_MOPS_F32", 0.0) * 512 for e in es)
        ns = statistics.median(e["ns"] for e in es)
        busy = statistics.median(e.get("SQ_VALU_MFMA_BUSY_CYCLES", 0.0) for e in es)
        gui = statistics.median(e.get("GRBM_GUI_ACTIVE", 0.0) for e in es)
        tflops = flops / ns / 1e3 if ns else 0.0
        f32_tflops = f32 / ns / 1e3 if ns else 0.0
        out[name] = {"dispatches": len(es), "flops": flops, "us": ns / 1e3, "tflops": tflops,
                     "frac": tflops / BF16_PEAK_TFLOPS, "f32_flops": f32, "f32_frac": f32_tflops / F32_PEAK_TFLOPS,
                     "util": 100.0 * busy / (gui / xcds * simds) if gui else 0.0}
    return out


def _mfma_md(d: str, kernel_regex: str, simds: int, xcds: int) -> str:
    rows = ["| kernel | dispatches | bf16 MFMA GFLOP issued | us | TFLOP/s | of bf16 peak | fp32 MFMA GFLOP | "
            "of fp32 peak | MfmaUtil % |",
            "|---|---|---|---|---|---|---|---|---|"]
    for name, m in sorted(mfma_by_kernel(d, kernel_regex, simds, xcds).items(),
                          key=lambda kv: -(kv[1]["flops"] + kv[1]["f32_flops"])):
        rows.append(f"| `{name}` | {m['dispatches']} | {m['flops'] / 1e9:.2f} | {m['us']:.1f} | {m['tflops']:.1f} | "
                    f"{m['frac']:.3f} | {m['f32_flops'] / 1e9:.2f} | {m['f32_frac']:.3f} | {m['util']:.1f} |")
    return "\n".join(rows)


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
    t.add_argument("--calls-per-op", type=int, default=1,
                   help="dispatches of each matching kernel per launch of the op (segmented scans)")
    m = sub.add_parser("mfma")
    m.add_argument("dir")
    m.add_argument("--kernel", default="", help="only kernels whose name matches this regex")
    m.add_argument("--simds", type=int, default=1024, help="SIMDs of the device (MI355X: 256 CUs x 4)")
    m.add_argument("--xcds", type=int, default=8, help="XCDs whose GRBM_GUI_ACTIVE counts are summed")
    a = p.parse_args(argv)
    if a.cmd == "stats":
        print(_stats_md(a.dir, a.kernel))
    elif a.cmd == "mfma":
        print(_mfma_md(a.dir, a.kernel, a.simds, a.xcds))
    else:
        print(_traffic_md(a))


if __name__ == "__main__":
    main()
