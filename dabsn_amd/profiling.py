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

    python -m dabsn_amd.profiling <results.db> [--top N] [--match REGEX] [--tail MARKER:N]
    python -m dabsn_amd.profiling <results.db> --categories STEPS
    python -m dabsn_amd.profiling --pmc-summary <dir> [--match REGEX]
    python -m dabsn_amd.profiling --mfma-dispatches <dir>
    python -m dabsn_amd.profiling --copy-probe <MiB>
    python -m dabsn_amd.profiling --gemm-shapes
    python -m dabsn_amd.profiling --pmc-json <out.json> --fetch <dir> --write <dir> \
        --copy-fetch <dir> --copy-write <dir> --copy-mib 512 --batch B --seq T --state H --chunk C

``pmc_json`` turns the four counter runs (FETCH_SIZE and WRITE_SIZE on the core scan kernels
and on the copy probe) into the per-launch HBM traffic file bench.py reports as
``roofline.traffic``: counter KiB per dispatch scaled to bytes by the copy probe's known size.
"""

from __future__ import annotations

import argparse
import re
import sqlite3
from collections import defaultdict


def kernel_stats(db_path: str, match: str | None = None,
                 tail: tuple[str, int] | None = None) -> list[dict[str, object]]:
    """Per-kernel statistics of a trace. ``tail = (marker, n)`` keeps only the dispatches
    between the end of the (n+1)-th last dispatch whose name matches ``marker`` and the end
    of the last one: the last n repetitions of a step that launches the marker once (e.g.
    the timed steps of a benchmark after its warm-up and set-up)."""
    con = sqlite3.connect(db_path)
    rows = con.execute("select name, duration, start, end from kernels order by start").fetchall()
    con.close()
    if tail is not None:
        marker, n = re.compile(tail[0]), int(tail[1])
        ends = [e for name, _, _, e in rows if marker.search(name)]
        if len(ends) <= n:
            raise ValueError(f"trace has {len(ends)} dispatches matching {tail[0]!r}, need {n + 1}")
        lo, hi = ends[-n - 1], ends[-1]
        rows = [r for r in rows if r[2] >= lo and r[3] <= hi]
    pattern = re.compile(match) if match else None
    agg: dict[str, list[int]] = defaultdict(list)
    for name, duration, _, _ in rows:
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


# Kernel categories of the scan+read step (first matching rule wins).
CATEGORIES = (
    ("core reverse scans", r"core_bwd_kernel"),
    ("core forward scans", r"core_fwd_kernel"),
    ("read GEMMs (gemm.hpp)", r"dabsn::gemm::gemm_kernel"),
    ("read row kernels (softmax, grad rows/tiles, reductions, ranges)",
     r"read3::(softmax_fwd|grad_rows|grad_tile|reduce_|ranges)"),
    ("read transposes", r"transpose_kernel"),
    ("hipBLASLt (read output projection, grad [Ug;A])", r"^(Custom_)?Cijk|^_UIOFGRO|^AV_"),
    ("long scan fwd+bwd", r"longmem::"),
    ("read glue (stats, normalise, select, gather, slot glue, read output)",
     r"dabsn::glue::|glue_|read_out|means_glue"),
    ("torch elementwise, copies, fills, reductions", r"at::native|rocclr"),
)


def categories(stats: list[dict[str, object]], steps: int) -> str:
    """Milliseconds per step by kernel category (``CATEGORIES``), from ``kernel_stats``."""
    total: dict[str, float] = defaultdict(float)
    for r in stats:
        cat = next((c for c, rx in CATEGORIES if re.search(rx, r["name"])), "other")
        total[cat] += r["total_ms"] / steps
    lines = ["| category | ms / step |", "|---|---|"]
    for cat, ms in sorted(total.items(), key=lambda kv: -kv[1]):
        lines.append(f"| {cat} | {ms:.2f} |")
    lines.append(f"| **sum of kernel durations** | **{sum(total.values()):.2f}** |")
    return "\n".join(lines)


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


def mfma_dispatches(directory: str, cus: int = 256, simds_per_cu: int = 4,
                    xcds: int = 8) -> list[dict[str, object]]:
    """Per dispatch of a ``--pmc SQ_INSTS_VALU_MFMA_MOPS_BF16 SQ_VALU_MFMA_BUSY_CYCLES
    GRBM_GUI_ACTIVE`` run, in dispatch order: bf16 MFMA flops (512 per MOPS unit), MFMA
    utilisation = busy SIMD cycles / (GRBM_GUI_ACTIVE / xcds x SIMDs) and the profiled
    duration."""
    import csv
    import glob
    rows: dict[int, dict[str, object]] = {}
    for path in glob.glob(f"{directory}/**/*counter_collection.csv", recursive=True):
        with open(path, newline="") as fh:
            for r in csv.DictReader(fh):
                d = rows.setdefault(int(r["Dispatch_Id"]), {
                    "kernel": r["Kernel_Name"], "grid": int(r["Grid_Size"]),
                    "ms": (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e6})
                d[r["Counter_Name"]] = float(r["Counter_Value"])
    out = []
    for did in sorted(rows):
        d = rows[did]
        busy = d.get("SQ_VALU_MFMA_BUSY_CYCLES", 0.0)
        active = d.get("GRBM_GUI_ACTIVE", 0.0) / xcds * cus * simds_per_cu
        flops = 512.0 * d.get("SQ_INSTS_VALU_MFMA_MOPS_BF16", 0.0)
        out.append({"dispatch": did, "kernel": d["kernel"], "grid": d["grid"], "ms": d["ms"],
                    "tflop": flops / 1e12, "busy": busy, "active": active,
                    "util": busy / active if active else 0.0})
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


def gemm_shapes(reps: int = 10) -> list[tuple[str, float, float]]:
    """hipBLASLt (through torch.bmm) on the full shapes of the three-way read's GEMMs for the
    last 1,024-query chunk of config 4 (16 batch rows, 4,096 bank slots, width 2,048, bf16
    operands): (name, ms per launch, TFLOP/s), ``reps`` timed launches after one warm-up."""
    import torch

    B, T, N, H = 16, 1024, 4096, 2048
    g = torch.Generator(device="cuda").manual_seed(0)
    q = torch.randn(B, T, H, device="cuda", generator=g).bfloat16()
    kt = torch.randn(B, H, N, device="cuda", generator=g).bfloat16()
    p = torch.randn(B, T, N, device="cuda", generator=g).bfloat16()
    v = torch.randn(B, N, H, device="cuda", generator=g).bfloat16()
    cases = [("S = Q K^T, bf16 out", lambda: torch.bmm(q, kt)),
             ("S = Q K^T, fp32 out", lambda: torch.bmm(q, kt, out_dtype=torch.float32)),
             ("O = P V, bf16 out", lambda: torch.bmm(p, v)),
             ("gK = G^T Q, left operand a transposed view", lambda: torch.bmm(p.transpose(1, 2), q))]
    flops = 2.0 * B * T * N * H
    out = []
    for name, fn in cases:
        fn()
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(reps):
            fn()
        b.record()
        torch.cuda.synchronize()
        ms = a.elapsed_time(b) / reps
        out.append((name, ms, flops / ms / 1e9))
    return out


# Core scan kernels by the names bench.py reports them under.
_CORE_KERNELS = {"core_fwd_kernel": "core_scan_fwd", "core_bwd_kernel": "core_scan_bwd"}


def _one(rows: list[dict[str, object]], counter: str, match: str) -> dict[str, object]:
    hits = [r for r in rows if r["counter"] == counter and re.search(match, r["kernel"])]
    if len(hits) != 1:
        raise SystemExit(f"expected one {counter} entry for {match!r}, found {len(hits)}")
    return hits[0]


def pmc_json(out: str, fetch_dir: str, write_dir: str, copy_fetch_dir: str, copy_write_dir: str,
             copy_mib: int, workload: dict[str, object]) -> dict[str, object]:
    """Per-launch HBM traffic of the core scan kernels, calibrated on the copy probe."""
    import json

    nbytes = copy_mib * 1024 * 1024
    cf = _one(pmc_summary(copy_fetch_dir), "FETCH_SIZE", "neg")["mean"]
    cw = _one(pmc_summary(copy_write_dir), "WRITE_SIZE", "neg")["mean"]
    ff, wf = nbytes / (cf * 1024.0), nbytes / (cw * 1024.0)
    fetch, write = pmc_summary(fetch_dir), pmc_summary(write_dir)
    kernels = {}
    for sym, name in _CORE_KERNELS.items():
        try:
            f, w = _one(fetch, "FETCH_SIZE", sym), _one(write, "WRITE_SIZE", sym)
        except SystemExit:
            continue
        fb, wb = f["mean"] * 1024.0 * ff, w["mean"] * 1024.0 * wf
        kernels[name] = {"kernel_symbol": f["kernel"], "fetch_size_kib": round(f["mean"], 1),
                         "write_size_kib": round(w["mean"], 1), "fetch_bytes": int(fb),
                         "write_bytes": int(wb), "traffic_bytes": int(fb + wb),
                         "dispatches": int(f["dispatches"])}
    doc = {"workload": workload,
           "copy_calibration": {"bytes_read_and_written": nbytes, "fetch_size_kib": round(cf, 1),
                                "write_size_kib": round(cw, 1), "fetch_factor": round(ff, 5),
                                "write_factor": round(wf, 5)},
           "kernels": kernels}
    with open(out, "w") as fh:
        json.dump(doc, fh, indent=1)
        fh.write("\n")
    return doc


def _dispatch_counters(directory: str) -> dict[int, dict[str, object]]:
    """Dispatch id -> (kernel, queue, counter value) of a single-counter rocprofv3 CSV run."""
    import csv
    from pathlib import Path

    out: dict[int, dict[str, object]] = {}
    for path in sorted(Path(directory).rglob("*counter_collection.csv")):
        with open(path, newline="") as fh:
            for r in csv.DictReader(fh):
                out[int(r["Dispatch_Id"])] = {"kernel": r["Kernel_Name"], "queue": int(r["Queue_Id"]),
                                              "value": float(r["Counter_Value"])}
    return out


def _short(name: str) -> str:
    return re.sub(r"^dabsn::", "", re.sub(r"\(.*", "", name).replace("void ", ""))


def step_traffic(fetch_dir: str, write_dir: str, copy_fetch_dir: str, copy_write_dir: str,
                 copy_mib: int, trace_db: str, match: str, scans_per_step: int) -> str:
    """Markdown tables of the HBM traffic of the last traced step: FETCH_SIZE and
    WRITE_SIZE per dispatch (copy-calibrated) from two counter runs of the bench, durations
    from a kernel-trace run of the same bench (dispatches of the step paired with trace
    records by kernel name and order). The step starts at its first forward-scan
    dispatch (``scans_per_step`` per step); the whole-device stream is the queue of the
    step's last statistics kernel."""
    import sqlite3

    nbytes = copy_mib * 1024 * 1024
    ff = nbytes / (_one(pmc_summary(copy_fetch_dir), "FETCH_SIZE", "neg")["mean"] * 1024.0)
    wf = nbytes / (_one(pmc_summary(copy_write_dir), "WRITE_SIZE", "neg")["mean"] * 1024.0)
    fe, wr = _dispatch_counters(fetch_dir), _dispatch_counters(write_dir)
    ids = sorted(fe)
    fwd = [i for i in ids if "core_fwd_kernel" in str(fe[i]["kernel"])]
    step = [i for i in ids if i >= fwd[-scans_per_step]]
    rx = re.compile(match)
    con = sqlite3.connect(trace_db)
    rows = [r for r in con.execute("select name, start, end from kernels order by start")
            if rx.search(r[0])]
    tf = [k for k, r in enumerate(rows) if "core_fwd_kernel" in r[0]]
    durations: dict[str, list[float]] = defaultdict(list)
    for name, start, end in rows[tf[-scans_per_step]:]:
        durations[_short(name)].append((end - start) / 1e3)
    seen: dict[str, int] = defaultdict(int)
    recs = []
    for i in step:
        n = _short(str(fe[i]["kernel"]))
        k = seen[n]
        seen[n] += 1
        d = durations[n][k] if k < len(durations[n]) else float("nan")
        f = float(fe[i]["value"]) * 1024.0 * ff
        w = float(wr[i]["value"]) * 1024.0 * wf if i in wr else float("nan")
        recs.append((i, n, int(fe[i]["queue"]), f, w, d))
    whole = [q for _, n, q, *_ in recs if n.startswith("glue::stats_kernel")][-1]
    lines = [f"calibration: fetch factor {ff:.5f}, write factor {wf:.5f}", "",
             "| # | kernel | FETCH MB | WRITE MB | traffic MB | us | GB/s | frac of 8 TB/s |",
             "|---|---|---|---|---|---|---|---|"]
    for i, n, q, f, w, d in recs:
        if q != whole:
            continue
        t = (f + w) / 1e6
        lines.append(f"| {i} | `{n[:70]}` | {f / 1e6:.1f} | {w / 1e6:.1f} | {t:.1f} | {d:.0f} | "
                     f"{t / d * 1e3:.0f} | {t / d * 1e3 / 8000:.3f} |")
    lines += ["", "| kernel | launches | FETCH MB | WRITE MB | us | GB/s |",
              "|---|---|---|---|---|---|"]
    agg: dict[str, list[float]] = defaultdict(lambda: [0, 0.0, 0.0, 0.0])
    for _, n, q, f, w, d in recs:
        if q == whole or "core_" in n:
            continue
        a = agg[n]
        a[0] += 1
        a[1] += f
        a[2] += w
        a[3] += d
    for n, (c, f, w, d) in sorted(agg.items(), key=lambda kv: -kv[1][3]):
        lines.append(f"| `{n[:70]}` | {int(c)} | {f / 1e6:.0f} | {w / 1e6:.0f} | {d:.0f} | "
                     f"{(f + w) / 1e6 / d * 1e3:.0f} |")
    return "\n".join(lines)


def main() -> None:
    p = argparse.ArgumentParser()
    p.add_argument("db", nargs="?")
    p.add_argument("--top", type=int, default=25)
    p.add_argument("--match", default=None)
    p.add_argument("--tail", default=None, metavar="MARKER:N",
                   help="only the last N repetitions of a step launching MARKER once")
    p.add_argument("--categories", type=int, default=None, metavar="STEPS",
                   help="milliseconds per step by kernel category, the trace holding STEPS steps")
    p.add_argument("--pmc-summary", default=None)
    p.add_argument("--mfma-dispatches", default=None, metavar="DIR",
                   help="per-dispatch MFMA flops and utilisation of a counter run")
    p.add_argument("--copy-probe", type=int, default=None)
    p.add_argument("--gemm-shapes", action="store_true",
                   help="hipBLASLt on the read GEMM shapes of the last config-4 chunk")
    p.add_argument("--pmc-json", default=None)
    p.add_argument("--step-traffic", default=None, metavar="TRACE_DB",
                   help="per-dispatch HBM traffic of the last traced step (with --fetch, --write, "
                        "--copy-fetch, --copy-write, --match)")
    for k in ("fetch", "write", "copy-fetch", "copy-write"):
        p.add_argument(f"--{k}", default=None)
    p.add_argument("--copy-mib", type=int, default=512)
    for k, d in (("batch", 16), ("seq", 4096), ("state", 2048), ("chunk", 1024)):
        p.add_argument(f"--{k}", type=int, default=d)
    p.add_argument("--dtype", default="bf16")
    args = p.parse_args()
    if args.step_traffic:
        from dabsn_amd.kernels.pipeline import windows

        print(step_traffic(args.fetch, args.write, args.copy_fetch, args.copy_write, args.copy_mib,
                           args.step_traffic,
                           args.match or "read3|glue|longmem|xpose|gemm_kernel|read_out|core_",
                           len(windows(args.seq, args.chunk))))
    elif args.pmc_json:
        doc = pmc_json(args.pmc_json, args.fetch, args.write, args.copy_fetch, args.copy_write,
                       args.copy_mib, {"batch": args.batch, "seq_len": args.seq,
                                       "state": args.state, "chunk_t": args.chunk,
                                       "dtype": args.dtype})
        for name, k in doc["kernels"].items():
            print(f"{name}: {k['traffic_bytes'] / 1e9:.3f} GB per launch "
                  f"({k['dispatches']} dispatches)")
    elif args.copy_probe:
        copy_probe(args.copy_probe)
    elif args.gemm_shapes:
        for name, ms, tf in gemm_shapes():
            print(f"{name:45s} {ms:.3f} ms {tf:.0f} TFLOP/s")
    elif args.mfma_dispatches:
        rows = mfma_dispatches(args.mfma_dispatches)
        print("| dispatch | output | grid | TFLOP | MFMA busy cycles | util | ms (profiled) | TFLOP/s |")
        print("|---|---|---|---|---|---|---|---|")
        for r in rows:
            outt = "fp32" if ", float," in r["kernel"] else "bf16"
            print(f"| {r['dispatch']} | {outt} | {r['grid']} | {r['tflop']:.3f} | {r['busy']:.3e} | "
                  f"{r['util']:.3f} | {r['ms']:.3f} | {r['tflop'] / r['ms'] * 1e3 if r['ms'] else 0:.0f} |")
        busy = sum(r["busy"] for r in rows)
        active = sum(r["active"] for r in rows)
        print(f"\n{len(rows)} dispatches: {sum(r['tflop'] for r in rows):.2f} TFLOP, MFMA utilisation "
              f"{busy / active if active else 0:.3f} (busy-cycle weighted)")
    elif args.pmc_summary:
        for r in pmc_summary(args.pmc_summary, args.match):
            name = r["kernel"] if len(r["kernel"]) <= 90 else r["kernel"][:87] + "..."
            print(f"{r['counter']:>12} {r['mean']:16.1f} {r['dispatches']:6d}  {name}")
    else:
        tail = None
        if args.tail:
            marker, _, n = args.tail.rpartition(":")
            tail = (marker, int(n))
        stats = kernel_stats(args.db, args.match, tail)
        if args.categories:
            print(categories(stats, args.categories))
        else:
            print(format_table(stats, args.top))


if __name__ == "__main__":
    main()
