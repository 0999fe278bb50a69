"""CPU baseline leg of bench.py: the reference SPINNV2 C runtime
(oracle/_ref/libspkv2_ref.so, built from /root/reference/runtime by
oracle/Makefile) timed on the host cores with the reference benchmark
protocol (runtime/tools/spkv2_bench.c:97-117: set_input outside the clock,
CLOCK_MONOTONIC around spkv2_run only) and its statistics
(spkv2_bench.c:136-159: min / avg / p50 = sorted[runs/2] /
p90 = sorted[runs*9/10] / max, in ms).

TEST AND BASELINE INFRASTRUCTURE ONLY: bench.py's cpu_baseline leg; the
product never loads the reference runtime.

Runs in its own process so OMP_NUM_THREADS applies to the reference's
OpenMP runtime.  Prints one JSON line.

    python -m oracle.cpu_baseline --model resnet101 --batch 1 --profile cpu_generic --runs 1
    python -m oracle.cpu_baseline --profile cpu_generic_nobnns --runs 20 --warmup 1 --max-seconds 20
"""

from __future__ import annotations

import argparse
import json
import os
import time


def host_cpu() -> dict:
    """nproc and the CPU model name (what `lscpu` prints as Model name)."""
    model = ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        nproc = len(os.sched_getaffinity(0))
    except AttributeError:  # pragma: no cover
        nproc = os.cpu_count() or 0
    return {"nproc": nproc, "cpu_model": model}


def stats_ms(times_s: list[float]) -> dict:
    """spkv2_bench.c:136-147"""
    t = sorted(x * 1e3 for x in times_s)
    n = len(t)
    return {"min_ms": t[0], "avg_ms": sum(t) / n, "p50_ms": t[n // 2], "p90_ms": t[(n * 9) // 10], "max_ms": t[-1]}


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--model", default="resnet101")
    ap.add_argument("--batch", type=int, default=1)
    ap.add_argument("--profile", default="cpu_generic")
    ap.add_argument("--runs", type=int, default=1)
    ap.add_argument("--warmup", type=int, default=0)
    ap.add_argument("--max-seconds", type=float, default=0.0,
                    help="stop the timed runs once they have taken this long (0: all --runs)")
    args = ap.parse_args()

    from spinnv2_amd.spk import models, write_spk

    from .ref_runtime import RefModel

    depth = int(args.model.replace("resnet", ""))
    g = models.resnet(depth, args.batch)
    blob = write_spk(g, args.profile)
    x = models.make_input(g.tensors[g.inputs[0]].shape)
    m = RefModel(blob)
    for _ in range(args.warmup):
        m.run(x)
    times = []
    out = None
    for _ in range(args.runs):
        # the reference bench sets the input before starting the clock
        m.set_input(0, x)
        t0 = time.perf_counter()
        rc = m.run_rc()
        times.append(time.perf_counter() - t0)
        if rc != 0:
            raise SystemExit(f"reference run failed: {rc}")
        if args.max_seconds and sum(times) >= args.max_seconds:
            break
    out = m.output(0)
    st = stats_ms(times)
    print(json.dumps({
        "model": args.model, "batch": args.batch, "profile": args.profile, "runs": len(times),
        "warmup": args.warmup, **st, "avg_s": st["avg_ms"] / 1e3, "images_per_sec": args.batch * 1e3 / st["avg_ms"],
        "threads": int(os.environ.get("OMP_NUM_THREADS", "0") or 0), **host_cpu(),
        "top1": int(out.reshape(args.batch, -1)[0].argmax()),
    }))


if __name__ == "__main__":
    main()
