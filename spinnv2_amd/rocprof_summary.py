"""Digests rocprofv3 CSV output into the short text summaries kept in profiles/.

    python -m spinnv2_amd.rocprof_summary stats   <kernel_stats.csv> --runs N [--match conv_igemm_i8]
           [--group NAME --include SUBSTR [--include ...] [--exclude SUBSTR ...]]
    python -m spinnv2_amd.rocprof_summary traffic --fetch <pmc.csv> --write <pmc.csv>
           --copy-fetch <pmc.csv> --copy-write <pmc.csv> --copy-bytes B --runs N --match conv_igemm
           [--group NAME --include SUBSTR [--include ...] [--exclude SUBSTR ...]]
    python -m spinnv2_amd.rocprof_summary mfma <pmc.csv> --runs N --match conv_igemm --cus 256 --xcds 8
           [--mops SQ_INSTS_VALU_MFMA_MOPS_I8 --peak 5000]
    python -m spinnv2_amd.rocprof_summary launches <kernel_trace.csv> --runs N [--match conv_igemm_i8]

`stats` divides rocprofv3 --kernel-trace --stats totals by the number of
spkv2_run calls the profiled command made (N), giving per-run kernel time;
--group totals the kernels whose name contains any --include and none of
the --exclude substrings (e.g. every launch of the conv nodes: the GEMM,
split-K epilogue and padding kernels, without the classifier Gemm's).
`traffic` sums FETCH_SIZE and WRITE_SIZE (KiB per dispatch) over the
kernels whose name contains --match (or the --group members), per run, and
scales each counter by bytes / counter of a plain copy kernel of known size
profiled the same way;
per kernel it also gives the HBM GB/s those bytes make over the dispatches'
own durations (timestamps of the FETCH_SIZE pass).
`mfma` reads a --pmc pass of an MFMA work counter (--mops, default
SQ_INSTS_VALU_MFMA_MOPS_F32; every SQ_INSTS_VALU_MFMA_MOPS_* counts in units
of 512 operations), SQ_VALU_MFMA_BUSY_CYCLES and GRBM_GUI_ACTIVE: per kernel
the MFMA operations the hardware counted, that work over the dispatches'
durations against --peak (T ops/s of the counted type; 157.3 for fp32, 5000
for int8), and MFMA busy cycles (per SIMD) over the
active cycles of all SIMDs: GRBM_GUI_ACTIVE / XCDs x CUs x 4 (on MI355X
GRBM_GUI_ACTIVE sums the 8 XCDs' counts: about 8 x duration x clock).
`launches` reads a --kernel-trace dispatch list and splits each kernel (name
containing --match) by its launch shape (workgroups x grid y x grid z, and
the workgroup size): the layers that share one tile configuration apart,
with dispatches per run, the median dispatch duration and time per run.
"""

from __future__ import annotations

import argparse
import csv
import re
from collections import defaultdict


def short_name(name: str) -> str:
    name = name.replace("spk::kern::", "").replace("(anonymous namespace)::", "").replace("void ", "")
    return re.sub(r"\(.*\)$", "", name)


def stats(path: str, runs: int, match: str | None = None, group: str | None = None,
          include: list[str] | None = None, exclude: list[str] | None = None) -> str:
    rows = list(csv.DictReader(open(path)))
    total = sum(float(r["TotalDurationNs"]) for r in rows)
    out = [f"{'kernel':48s} {'calls/run':>9s} {'avg us':>9s} {'ms/run':>9s} {'share':>7s}"]
    for r in sorted(rows, key=lambda r: -float(r["TotalDurationNs"])):
        t = float(r["TotalDurationNs"])
        out.append(f"{short_name(r['Name'])[:48]:48s} {int(r['Calls']) / runs:9.1f} {float(r['AverageNs']) / 1e3:9.2f} "
                   f"{t / runs / 1e6:9.3f} {100 * t / total:6.1f}%")
    out.append(f"{'all kernels':48s} {'':9s} {'':9s} {total / runs / 1e6:9.3f}")
    if match:
        sel = [r for r in rows if match in r["Name"]]
        ms = sum(float(r["TotalDurationNs"]) for r in sel) / runs / 1e6
        calls = sum(int(r["Calls"]) for r in sel) / runs
        out.append("")
        out.append(f"result {match}_ms_per_run = {ms:.6f}")
        out.append(f"result {match}_calls_per_run = {calls:.1f}")
    if group:
        inc, exc = include or [], exclude or []
        sel = [r for r in rows if any(s in short_name(r["Name"]) for s in inc)
               and not any(s in short_name(r["Name"]) for s in exc)]
        ms = sum(float(r["TotalDurationNs"]) for r in sel) / runs / 1e6
        calls = sum(int(r["Calls"]) for r in sel) / runs
        out.append("")
        out.append(f"group {group}: names containing any of {inc}" + (f", none of {exc}" if exc else ""))
        out.append(f"result {group}_ms_per_run = {ms:.6f}")
        out.append(f"result {group}_calls_per_run = {calls:.1f}")
    return "\n".join(out)


def _counter_per_kernel(path: str) -> dict[str, list[float]]:
    agg: dict[str, list[float]] = defaultdict(lambda: [0, 0.0])
    for r in csv.DictReader(open(path)):
        a = agg[r["Kernel_Name"]]
        a[0] += 1
        a[1] += float(r["Counter_Value"])
    return agg


def _durations_per_kernel(path: str) -> dict[str, float]:
    """Summed dispatch durations (ns) per kernel, each dispatch once."""
    seen: dict[str, float] = {}
    per: dict[str, float] = defaultdict(float)
    for r in csv.DictReader(open(path)):
        d = r["Dispatch_Id"]
        if d in seen:
            continue
        seen[d] = 1.0
        per[r["Kernel_Name"]] += float(r["End_Timestamp"]) - float(r["Start_Timestamp"])
    return per


def _copy_scale(path: str, copy_bytes: int) -> float:
    vals = [float(r["Counter_Value"]) for r in csv.DictReader(open(path)) if "copy_kernel" in r["Kernel_Name"]]
    if not vals:
        raise SystemExit(f"no copy_kernel dispatch in {path}")
    return copy_bytes / (sum(vals) / len(vals) * 1024.0)


def _member(name: str, match: str | None, include: list[str], exclude: list[str]) -> bool:
    """A kernel of the totalled set: any --include (and no --exclude) when
    includes are given, else a name containing --match."""
    n = short_name(name)
    if include:
        return any(s in n for s in include) and not any(s in n for s in exclude)
    return bool(match) and match in name


def traffic(args) -> str:
    include, exclude = getattr(args, "include", None) or [], getattr(args, "exclude", None) or []
    fs = _copy_scale(args.copy_fetch, args.copy_bytes)
    ws = _copy_scale(args.copy_write, args.copy_bytes)
    fetch = _counter_per_kernel(args.fetch)
    write = _counter_per_kernel(args.write)
    dur = _durations_per_kernel(args.fetch)
    out = [f"copy kernel {args.copy_bytes} B: bytes per FETCH_SIZE KiB-unit x{fs:.4f} / 1024, "
           f"per WRITE_SIZE KiB-unit x{ws:.4f} / 1024",
           f"{'kernel':48s} {'disp/run':>8s} {'read MB/run':>12s} {'write MB/run':>12s} {'HBM GB/s':>9s}"]
    tot_r = tot_w = 0.0
    disp = 0
    for name in sorted(set(fetch) | set(write), key=lambda n: -fetch.get(n, [0, 0])[1]):
        rd = fetch.get(name, [0, 0.0])[1] * 1024 * fs / args.runs
        wr = write.get(name, [0, 0.0])[1] * 1024 * ws / args.runs
        ns = dur.get(name, 0.0) / args.runs
        gbps = (rd + wr) / ns if ns > 0 else 0.0
        out.append(f"{short_name(name)[:48]:48s} {fetch.get(name, [0])[0] / args.runs:8.1f} {rd / 1e6:12.1f} "
                   f"{wr / 1e6:12.1f} {gbps:9.0f}")
        if _member(name, args.match, include, exclude):
            tot_r += rd
            tot_w += wr
            disp += fetch.get(name, [0])[0]
    label = getattr(args, "group", None) or args.match
    out.append("")
    if include:
        out.append(f"group {label}: names containing any of {include}" + (f", none of {exclude}" if exclude else ""))
    out.append(f"result {label}_read_bytes_per_step = {tot_r:.0f}")
    out.append(f"result {label}_write_bytes_per_step = {tot_w:.0f}")
    out.append(f"result conv_hbm_bytes_per_step = {tot_r + tot_w:.0f}")
    out.append(f"result conv_dispatches_per_step = {disp / args.runs:.0f}")
    return "\n".join(out)


def mfma(args) -> str:
    per: dict[str, dict[str, float]] = defaultdict(lambda: defaultdict(float))
    seen = set()
    for r in csv.DictReader(open(args.csv)):
        k = per[r["Kernel_Name"]]
        k[r["Counter_Name"]] += float(r["Counter_Value"])
        if r["Dispatch_Id"] not in seen:
            seen.add(r["Dispatch_Id"])
            k["ns"] += float(r["End_Timestamp"]) - float(r["Start_Timestamp"])
            k["n"] += 1
    op = "OP" if args.mops.endswith("I8") else "FLOP"  # integer MFMA work is counted in operations
    out = [f"{'kernel':48s} {'disp/run':>8s} {'avg us':>8s} {'G' + op + '/run':>10s} {'T' + op + '/s':>8s} "
           f"{'% peak':>7s} {'busy %':>7s}"]
    tot_f = tot_ns = tot_busy = tot_active = 0.0
    for name, k in sorted(per.items(), key=lambda kv: -kv[1]["ns"]):
        if args.match not in name:
            continue
        flop = k[args.mops] * 512
        tf = flop / k["ns"] / 1e3 if k["ns"] else 0.0
        simd_cycles = k["GRBM_GUI_ACTIVE"] / args.xcds * args.cus * 4
        busy = k["SQ_VALU_MFMA_BUSY_CYCLES"] / simd_cycles if simd_cycles else 0.0
        out.append(f"{short_name(name)[:48]:48s} {k['n'] / args.runs:8.1f} {k['ns'] / k['n'] / 1e3:8.2f} "
                   f"{flop / args.runs / 1e9:10.1f} {tf:8.1f} {100 * tf / args.peak:6.1f}% {100 * busy:6.1f}%")
        tot_f += flop
        tot_ns += k["ns"]
        tot_busy += k["SQ_VALU_MFMA_BUSY_CYCLES"]
        tot_active += k["GRBM_GUI_ACTIVE"]
    tf = tot_f / tot_ns / 1e3 if tot_ns else 0.0
    out.append("")
    out.append(f"result {args.match}_mfma_flop_per_run = {tot_f / args.runs:.0f}")
    out.append(f"result {args.match}_mfma_tflops = {tf:.2f}")
    out.append(f"result {args.match}_mfma_frac_of_peak = {tf / args.peak:.4f}")
    simd_cycles = tot_active / args.xcds * args.cus * 4
    out.append(f"result {args.match}_mfma_busy_frac = {tot_busy / simd_cycles if simd_cycles else 0:.4f}")
    return "\n".join(out)


def launches(path: str, runs: int, match: str | None = None) -> str:
    per: dict[tuple, list[float]] = defaultdict(list)
    for r in csv.DictReader(open(path)):
        name = short_name(r["Kernel_Name"])
        if match and match not in r["Kernel_Name"]:
            continue
        wg = int(r["Workgroup_Size_X"]) * int(r["Workgroup_Size_Y"]) * int(r["Workgroup_Size_Z"])
        shape = (int(r["Grid_Size_X"]) // max(int(r["Workgroup_Size_X"]), 1), int(r["Grid_Size_Y"]),
                 int(r["Grid_Size_Z"]), wg)
        per[(name, shape)].append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
    out = [f"{'kernel':44s} {'workgroups':>16s} {'threads':>7s} {'disp/run':>8s} {'median us':>9s} {'ms/run':>8s}"]
    for (name, (gx, gy, gz, wg)), d in sorted(per.items(), key=lambda kv: -sum(kv[1])):
        d = sorted(d)
        med = d[len(d) // 2] if len(d) % 2 else (d[len(d) // 2 - 1] + d[len(d) // 2]) / 2
        out.append(f"{name[:44]:44s} {f'{gx}x{gy}x{gz}':>16s} {wg:7d} {len(d) / runs:8.1f} {med:9.2f} "
                   f"{sum(d) / runs / 1e3:8.3f}")
    return "\n".join(out)


def main() -> None:
    ap = argparse.ArgumentParser()
    sub = ap.add_subparsers(dest="cmd", required=True)
    s = sub.add_parser("stats")
    s.add_argument("csv")
    s.add_argument("--runs", type=int, required=True)
    s.add_argument("--match", default=None, help="also total the kernels whose name contains this")
    s.add_argument("--group", default=None, help="name of a kernel group totalled from --include / --exclude")
    s.add_argument("--include", action="append", default=[], help="group member: name contains this")
    s.add_argument("--exclude", action="append", default=[], help="not a group member: name contains this")
    t = sub.add_parser("traffic")
    for k in ("fetch", "write", "copy_fetch", "copy_write"):
        t.add_argument("--" + k.replace("_", "-"), dest=k, required=True)
    t.add_argument("--copy-bytes", type=int, required=True)
    t.add_argument("--runs", type=int, required=True)
    t.add_argument("--match", default="conv_igemm")
    t.add_argument("--group", default=None, help="label of the kernels totalled from --include / --exclude")
    t.add_argument("--include", action="append", default=[], help="totalled: name contains this")
    t.add_argument("--exclude", action="append", default=[], help="not totalled: name contains this")
    m = sub.add_parser("mfma")
    m.add_argument("csv")
    m.add_argument("--runs", type=int, required=True)
    m.add_argument("--match", default="conv_igemm")
    m.add_argument("--cus", type=int, default=256)
    m.add_argument("--xcds", type=int, default=8)
    m.add_argument("--peak", type=float, default=157.3, help="T ops/s of the counted MFMA type (fp32: 157.3)")
    m.add_argument("--mops", default="SQ_INSTS_VALU_MFMA_MOPS_F32", help="MFMA work counter (units of 512 ops)")
    ln = sub.add_parser("launches")
    ln.add_argument("csv")
    ln.add_argument("--runs", type=int, required=True)
    ln.add_argument("--match", default=None, help="only kernels whose name contains this")
    a = ap.parse_args()
    print({"stats": lambda: stats(a.csv, a.runs, a.match, a.group, a.include, a.exclude), "traffic": lambda: traffic(a),
           "mfma": lambda: mfma(a), "launches": lambda: launches(a.csv, a.runs, a.match)}[a.cmd]())


if __name__ == "__main__":
    main()
