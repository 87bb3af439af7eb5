"""Summaries of rocprofv3 CSV output for the committed profiles.

    python -m gfxinfer_amd.rocprof_summary stats <dir> [--match NAME]...
    python -m gfxinfer_amd.rocprof_summary pmc <fetch_dir> <write_dir> --kernel NAME \\
        --copy NAME --copy-bytes N

    python -m gfxinfer_amd.rocprof_summary rounds <dir> --marker NAME --rounds N
    python -m gfxinfer_amd.rocprof_summary counters <dir>... --kernel NAME [--us T]
    python -m gfxinfer_amd.rocprof_summary shapes <dir> [--match NAME]...

`stats` prints the kernel table of a --kernel-trace --stats run (calls, total,
average, min, max per kernel).  `rounds` reads the kernel trace of such a run and
prints, for the last N rounds (a round starts at each dispatch of the marker
kernel), the span per round, the GPU-busy time per round and each kernel's time
and dispatch count per round.  `pmc` reads two --pmc runs (FETCH_SIZE, then
WRITE_SIZE; both in KiB per dispatch), calibrates each counter on the copy kernel
of known size (it reads and writes exactly N bytes) and prints the HBM bytes per
dispatch of the named kernel.  `shapes` splits a --kernel-trace run by launch
shape (kernel, grid, workgroup) and prints each shape's dispatch count and median and
minimum duration.  `counters` prints the per-dispatch median of every
counter that --pmc runs collected for the named kernel and, given the kernel's mean
duration T (from a --kernel-trace run), the derived figures: MFMA busy fraction
(SQ_VALU_MFMA_BUSY_CYCLES over 1024 SIMDs x T x 2.4 GHz), average DRAM read latency
(TCC_EA0_RDREQ_LEVEL / TCC_EA0_RDREQ, TCC cycles) and average DRAM reads in flight
(TCC_EA0_RDREQ_LEVEL / (T x 2.4 GHz), 128-byte requests).
"""
from __future__ import annotations

import argparse
import csv
import glob
import os
import statistics


def _csv(directory: str, suffix: str) -> list[dict]:
    paths = glob.glob(os.path.join(directory, "**", f"*{suffix}"), recursive=True)
    if not paths:
        raise SystemExit(f"no *{suffix} under {directory}")
    rows: list[dict] = []
    for p in paths:
        with open(p) as f:
            rows.extend(csv.DictReader(f))
    return rows


def short(name: str) -> str:
    name = name.replace("void ", "").replace("gfx950::(anonymous namespace)::", "")
    return name.split("(")[0]


def stats(directory: str, match: list[str]) -> str:
    rows = _csv(directory, "kernel_stats.csv")
    lines = [f"{'calls':>7} {'total_us':>11} {'avg_us':>9} {'min_us':>9} {'max_us':>9}  kernel"]
    for r in sorted(rows, key=lambda r: -float(r["TotalDurationNs"])):
        if match and not any(m in r["Name"] for m in match):
            continue
        lines.append(f"{int(r['Calls']):7d} {float(r['TotalDurationNs']) / 1e3:11.1f} "
                     f"{float(r['AverageNs']) / 1e3:9.3f} {float(r['MinNs']) / 1e3:9.3f} "
                     f"{float(r['MaxNs']) / 1e3:9.3f}  {short(r['Name'])}")
    return "\n".join(lines)


def rounds(directory: str, marker: str, count: int) -> str:
    rows = sorted(_csv(directory, "kernel_trace.csv"), key=lambda r: int(r["Start_Timestamp"]))
    starts = [i for i, r in enumerate(rows) if marker in r["Kernel_Name"]]
    if len(starts) < count:
        raise SystemExit(f"only {len(starts)} dispatches of {marker!r}")
    window = rows[starts[-count]:]
    total: dict[str, float] = {}
    calls: dict[str, int] = {}
    for r in window:
        name = short(r["Kernel_Name"])
        total[name] = total.get(name, 0.0) + (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3
        calls[name] = calls.get(name, 0) + 1
    span = (int(window[-1]["End_Timestamp"]) - int(window[0]["Start_Timestamp"])) / 1e3
    lines = [f"rounds {count}: span {span / count:.1f} us/round, GPU busy {sum(total.values()) / count:.1f} "
             f"us/round, {len(window) / count:.1f} dispatches/round",
             f"{'us/round':>9} {'calls/round':>11} {'avg_us':>8}  kernel"]
    for name, t in sorted(total.items(), key=lambda kv: -kv[1]):
        lines.append(f"{t / count:9.1f} {calls[name] / count:11.1f} {t / calls[name]:8.2f}  {name}")
    return "\n".join(lines)


def _per_dispatch(directory: str, counter: str, needle: str) -> list[float]:
    per: dict[int, float] = {}
    for r in _csv(directory, "counter_collection.csv"):
        if r["Counter_Name"] != counter or needle not in r["Kernel_Name"]:
            continue
        d = int(r["Dispatch_Id"])
        per[d] = per.get(d, 0.0) + float(r["Counter_Value"])
    return [per[d] for d in sorted(per)]


def pmc(fetch_dir: str, write_dir: str, kernel: str, copy: str, copy_bytes: int) -> str:
    out = []
    total = 0.0
    for counter, directory in (("FETCH_SIZE", fetch_dir), ("WRITE_SIZE", write_dir)):
        copy_kib = _per_dispatch(directory, counter, copy)
        kern_kib = _per_dispatch(directory, counter, kernel)
        if not copy_kib or not kern_kib:
            raise SystemExit(f"{counter}: missing dispatches of {copy!r} or {kernel!r}")
        factor = copy_bytes / max(copy_kib)  # bytes per counted KiB, from the copy
        value = statistics.median(kern_kib) * factor
        total += value
        out.append(f"{counter}: copy {max(copy_kib):.0f} KiB for {copy_bytes} B -> factor "
                   f"{factor:.1f} B per counted KiB; kernel median {statistics.median(kern_kib):.0f} KiB "
                   f"over {len(kern_kib)} dispatches -> {value:.0f} B")
    out.append(f"traffic_bytes_per_launch = {total:.0f}")
    return "\n".join(out)


def shapes(directory: str, match: list[str]) -> str:
    groups: dict[tuple, list[float]] = {}
    for r in _csv(directory, "kernel_trace.csv"):
        if match and not any(m in r["Kernel_Name"] for m in match):
            continue
        wg = int(r["Workgroup_Size_X"])
        key = (short(r["Kernel_Name"]), int(r["Grid_Size_X"]) // wg, wg)
        groups.setdefault(key, []).append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
    lines = [f"{'workgroups':>10} {'threads':>7} {'calls':>6} {'median_us':>9} {'min_us':>8}  kernel"]
    for (name, wgs, wg), v in sorted(groups.items()):
        lines.append(f"{wgs:10d} {wg:7d} {len(v):6d} {statistics.median(v):9.2f} {min(v):8.2f}  {name}")
    return "\n".join(lines)


SIMDS = 1024          # 256 CUs x 4 SIMDs
CLOCK_GHZ = 2.4       # MI355X peak engine clock


def counters(directories: list[str], kernel: str, us: float | None) -> str:
    names: set[str] = set()
    for d in directories:
        names.update(r["Counter_Name"] for r in _csv(d, "counter_collection.csv") if kernel in r["Kernel_Name"])
    med: dict[str, float] = {}
    lines = []
    for name in sorted(names):
        values = []
        for d in directories:
            values += _per_dispatch(d, name, kernel)
        med[name] = statistics.median(values)
        lines.append(f"{name:36s} median {med[name]:.6g} over {len(values)} dispatches")
    if us:
        cycles = us * 1e3 * CLOCK_GHZ
        if "SQ_VALU_MFMA_BUSY_CYCLES" in med:
            lines.append(f"mfma_busy_fraction = {med['SQ_VALU_MFMA_BUSY_CYCLES'] / (SIMDS * cycles):.4f}  "
                         f"(kernel {us} us)")
        if "TCC_EA0_RDREQ_LEVEL_sum" in med and "TCC_EA0_RDREQ_sum" in med:
            lines.append(f"dram_read_latency_cycles = {med['TCC_EA0_RDREQ_LEVEL_sum'] / med['TCC_EA0_RDREQ_sum']:.0f}")
            inflight = med["TCC_EA0_RDREQ_LEVEL_sum"] / cycles
            lines.append(f"dram_reads_in_flight = {inflight:.0f} ({inflight * 128 / 1e6:.2f} MB)")
    return "\n".join(lines)


def main() -> None:
    ap = argparse.ArgumentParser()
    sub = ap.add_subparsers(dest="cmd", required=True)
    a = sub.add_parser("stats")
    a.add_argument("directory")
    a.add_argument("--match", action="append", default=[])
    b = sub.add_parser("pmc")
    b.add_argument("fetch_dir")
    b.add_argument("write_dir")
    b.add_argument("--kernel", required=True)
    b.add_argument("--copy", required=True)
    b.add_argument("--copy-bytes", type=int, required=True)
    c = sub.add_parser("rounds")
    c.add_argument("directory")
    c.add_argument("--marker", required=True)
    c.add_argument("--rounds", type=int, required=True)
    d = sub.add_parser("counters")
    d.add_argument("directories", nargs="+")
    d.add_argument("--kernel", required=True)
    d.add_argument("--us", type=float, default=None)
    e = sub.add_parser("shapes")
    e.add_argument("directory")
    e.add_argument("--match", action="append", default=[])
    args = ap.parse_args()
    if args.cmd == "shapes":
        print(shapes(args.directory, args.match))
        return
    if args.cmd == "counters":
        print(counters(args.directories, args.kernel, args.us))
        return
    if args.cmd == "stats":
        print(stats(args.directory, args.match))
    elif args.cmd == "rounds":
        print(rounds(args.directory, args.marker, args.rounds))
    else:
        print(pmc(args.fetch_dir, args.write_dir, args.kernel, args.copy, args.copy_bytes))


if __name__ == "__main__":
    main()
