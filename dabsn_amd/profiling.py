"""Helpers for reading rocprofv3 output.

Kernel traces: ``rocprofv3 --stats`` normally writes a kernel_stats.csv; when the profiler
does not get that far (for example it can exit abnormally after the profiled program has
finished), the SQLite results database it wrote still holds every dispatch. ``kernel_stats``
reads the ``kernels`` view of that database: per kernel symbol, calls, total, average,
minimum and maximum duration.

Counters: ``pmc_summary`` averages each counter per dispatch and kernel over the
``*counter_collection.csv`` files of a ``rocprofv3 --pmc ... -f csv`` run. ``copy_probe``
launches a plain elementwise copy of known size (reads and writes ``mib`` MiB once per
launch), so the same counters read on it give the scale between counter units and bytes.

    python -m dabsn_amd.profiling <results.db> [--top N] [--match REGEX]
    python -m dabsn_amd.profiling --pmc-summary <dir> [--match REGEX]
    python -m dabsn_amd.profiling --copy-probe <MiB>
"""

from __future__ import annotations

import argparse
import re
import sqlite3
from collections import defaultdict


def kernel_stats(db_path: str, match: str | None = None) -> list[dict[str, object]]:
    con = sqlite3.connect(db_path)
    rows = con.execute("select name, duration from kernels").fetchall()
    con.close()
    pattern = re.compile(match) if match else None
    agg: dict[str, list[int]] = defaultdict(list)
    for name, duration in rows:
        if pattern and not pattern.search(name):
            continue
        agg[name].append(int(duration))
    out = []
    for name, durations in agg.items():
        total = sum(durations)
        out.append({"name": name, "calls": len(durations), "total_ms": total / 1e6,
                    "avg_ms": total / len(durations) / 1e6, "min_ms": min(durations) / 1e6,
                    "max_ms": max(durations) / 1e6})
    out.sort(key=lambda r: -r["total_ms"])
    return out


def format_table(stats: list[dict[str, object]], top: int) -> str:
    total = sum(r["total_ms"] for r in stats) or 1.0
    lines = [f"{'total_ms':>10} {'pct':>6} {'calls':>6} {'avg_ms':>10} {'min_ms':>10} {'max_ms':>10}  kernel"]
    for r in stats[:top]:
        name = r["name"] if len(r["name"]) <= 110 else r["name"][:107] + "..."
        lines.append(f"{r['total_ms']:10.3f} {100 * r['total_ms'] / total:5.1f}% {r['calls']:6d} "
                     f"{r['avg_ms']:10.4f} {r['min_ms']:10.4f} {r['max_ms']:10.4f}  {name}")
    return "\n".join(lines)


def pmc_summary(directory: str, match: str | None = None) -> list[dict[str, object]]:
    """Mean value per dispatch of every counter, per kernel, from rocprofv3 CSV output."""
    import csv
    from pathlib import Path

    pattern = re.compile(match) if match else None
    acc: dict[tuple[str, str], list[float]] = defaultdict(list)
    for path in sorted(Path(directory).rglob("*counter_collection.csv")):
        with open(path, newline="") as fh:
            for row in csv.DictReader(fh):
                name = row.get("Kernel_Name", "")
                if pattern and not pattern.search(name):
                    continue
                acc[(name, row.get("Counter_Name", ""))].append(float(row.get("Counter_Value", 0.0)))
    out = [{"kernel": k, "counter": c, "dispatches": len(v), "mean": sum(v) / len(v)}
           for (k, c), v in acc.items()]
    out.sort(key=lambda r: (r["counter"], -r["mean"]))
    return out


def copy_probe(mib: int, reps: int = 5) -> None:
    """Launch ``reps`` elementwise copies (torch.neg) that each read and write ``mib`` MiB."""
    import torch

    n = mib * 1024 * 1024 // 2
    src = torch.ones(n, device="cuda", dtype=torch.bfloat16)
    dst = torch.empty_like(src)
    for _ in range(reps):
        torch.neg(src, out=dst)
    torch.cuda.synchronize()
    print(f"copy probe: {reps} launches of neg over {mib} MiB bf16: "
          f"{n * 2} bytes read and {n * 2} bytes written per launch")


def main() -> None:
    p = argparse.ArgumentParser()
    p.add_argument("db", nargs="?")
    p.add_argument("--top", type=int, default=25)
    p.add_argument("--match", default=None)
    p.add_argument("--pmc-summary", default=None)
    p.add_argument("--copy-probe", type=int, default=None)
    args = p.parse_args()
    if args.copy_probe:
        copy_probe(args.copy_probe)
    elif args.pmc_summary:
        for r in pmc_summary(args.pmc_summary, args.match):
            name = r["kernel"] if len(r["kernel"]) <= 90 else r["kernel"][:87] + "..."
            print(f"{r['counter']:>12} {r['mean']:16.1f} {r['dispatches']:6d}  {name}")
    else:
        print(format_table(kernel_stats(args.db, args.match), args.top))


if __name__ == "__main__":
    main()
