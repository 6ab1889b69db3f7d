"""Summarise a ``rocprofv3 --kernel-trace`` results database into per-kernel statistics.

``rocprofv3 --stats`` normally writes a kernel_stats.csv; when the profiler does not get
that far (for example it can exit abnormally after the profiled program has finished),
the SQLite results database it wrote still holds every dispatch. This reads the
``kernels`` view of that database and prints, per kernel symbol: calls, total, average,
minimum and maximum duration.

    python -m dabsn_amd.profiling <results.db> [--top N] [--match REGEX]
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


def main() -> None:
    p = argparse.ArgumentParser()
    p.add_argument("db")
    p.add_argument("--top", type=int, default=25)
    p.add_argument("--match", default=None)
    args = p.parse_args()
    print(format_table(kernel_stats(args.db, args.match), args.top))


if __name__ == "__main__":
    main()
