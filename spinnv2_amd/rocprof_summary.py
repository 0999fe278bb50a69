"""Digests rocprofv3 CSV output into the short text summaries kept in profiles/.

    python -m spinnv2_amd.rocprof_summary stats   <kernel_stats.csv> --runs N
    python -m spinnv2_amd.rocprof_summary traffic --fetch <pmc.csv> --write <pmc.csv>
           --copy-fetch <pmc.csv> --copy-write <pmc.csv> --copy-bytes B --runs N --match conv_igemm

`stats` divides rocprofv3 --kernel-trace --stats totals by the number of
spkv2_run calls the profiled command made (N), giving per-run kernel time.
`traffic` sums FETCH_SIZE and WRITE_SIZE (KiB per dispatch) over the
kernels whose name contains --match, per run, and scales each counter by
bytes / counter of a plain copy kernel of known size profiled the same way.
"""

from __future__ import annotations

import argparse
import csv
import re
from collections import defaultdict


def short_name(name: str) -> str:
    name = name.replace("spk::kern::", "").replace("(anonymous namespace)::", "").replace("void ", "")
    return re.sub(r"\(.*\)$", "", name)


def stats(path: str, runs: int) -> str:
    rows = list(csv.DictReader(open(path)))
    total = sum(float(r["TotalDurationNs"]) for r in rows)
    out = [f"{'kernel':48s} {'calls/run':>9s} {'avg us':>9s} {'ms/run':>9s} {'share':>7s}"]
    for r in sorted(rows, key=lambda r: -float(r["TotalDurationNs"])):
        t = float(r["TotalDurationNs"])
        out.append(f"{short_name(r['Name'])[:48]:48s} {int(r['Calls']) / runs:9.1f} {float(r['AverageNs']) / 1e3:9.2f} "
                   f"{t / runs / 1e6:9.3f} {100 * t / total:6.1f}%")
    out.append(f"{'all kernels':48s} {'':9s} {'':9s} {total / runs / 1e6:9.3f}")
    return "\n".join(out)


def _counter_per_kernel(path: str) -> dict[str, list[float]]:
    agg: dict[str, list[float]] = defaultdict(lambda: [0, 0.0])
    for r in csv.DictReader(open(path)):
        a = agg[r["Kernel_Name"]]
        a[0] += 1
        a[1] += float(r["Counter_Value"])
    return agg


def _copy_scale(path: str, copy_bytes: int) -> float:
    vals = [float(r["Counter_Value"]) for r in csv.DictReader(open(path)) if "copy_kernel" in r["Kernel_Name"]]
    if not vals:
        raise SystemExit(f"no copy_kernel dispatch in {path}")
    return copy_bytes / (sum(vals) / len(vals) * 1024.0)


def traffic(args) -> str:
    fs = _copy_scale(args.copy_fetch, args.copy_bytes)
    ws = _copy_scale(args.copy_write, args.copy_bytes)
    fetch = _counter_per_kernel(args.fetch)
    write = _counter_per_kernel(args.write)
    out = [f"copy kernel {args.copy_bytes} B: bytes per FETCH_SIZE KiB-unit x{fs:.4f} / 1024, "
           f"per WRITE_SIZE KiB-unit x{ws:.4f} / 1024",
           f"{'kernel':48s} {'disp/run':>8s} {'read MB/run':>12s} {'write MB/run':>12s}"]
    tot_r = tot_w = 0.0
    disp = 0
    for name in sorted(set(fetch) | set(write), key=lambda n: -fetch.get(n, [0, 0])[1]):
        rd = fetch.get(name, [0, 0.0])[1] * 1024 * fs / args.runs
        wr = write.get(name, [0, 0.0])[1] * 1024 * ws / args.runs
        out.append(f"{short_name(name)[:48]:48s} {fetch.get(name, [0])[0] / args.runs:8.1f} {rd / 1e6:12.1f} "
                   f"{wr / 1e6:12.1f}")
        if args.match in name:
            tot_r += rd
            tot_w += wr
            disp += fetch.get(name, [0])[0]
    out.append("")
    out.append(f"result {args.match}_read_bytes_per_step = {tot_r:.0f}")
    out.append(f"result {args.match}_write_bytes_per_step = {tot_w:.0f}")
    out.append(f"result conv_hbm_bytes_per_step = {tot_r + tot_w:.0f}")
    out.append(f"result conv_dispatches_per_step = {disp / args.runs:.0f}")
    return "\n".join(out)


def main() -> None:
    ap = argparse.ArgumentParser()
    sub = ap.add_subparsers(dest="cmd", required=True)
    s = sub.add_parser("stats")
    s.add_argument("csv")
    s.add_argument("--runs", type=int, required=True)
    t = sub.add_parser("traffic")
    for k in ("fetch", "write", "copy_fetch", "copy_write"):
        t.add_argument("--" + k.replace("_", "-"), dest=k, required=True)
    t.add_argument("--copy-bytes", type=int, required=True)
    t.add_argument("--runs", type=int, required=True)
    t.add_argument("--match", default="conv_igemm")
    a = ap.parse_args()
    print(stats(a.csv, a.runs) if a.cmd == "stats" else traffic(a))


if __name__ == "__main__":
    main()
