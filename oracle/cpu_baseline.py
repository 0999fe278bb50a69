"""CPU baseline leg of bench.py: the reference SPINNV2 C runtime
(oracle/_ref/libspkv2_ref.so, built from /root/reference/runtime by
oracle/Makefile) timed on the host cores with the reference benchmark
protocol (runtime/tools/spkv2_bench.c:97-117: set_input outside the clock,
CLOCK_MONOTONIC around spkv2_run only).

Runs in its own process so OMP_NUM_THREADS applies to the reference's
OpenMP runtime.  Prints one JSON line.

    python -m oracle.cpu_baseline --model resnet101 --batch 1 --profile cpu_generic --runs 1
"""

from __future__ import annotations

import argparse
import json
import os
import time


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--model", default="resnet101")
    ap.add_argument("--batch", type=int, default=1)
    ap.add_argument("--profile", default="cpu_generic")
    ap.add_argument("--runs", type=int, default=1)
    ap.add_argument("--warmup", type=int, default=0)
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
        t0 = time.perf_counter()
        out = m.run(x)
        times.append(time.perf_counter() - t0)
    avg = sum(times) / len(times)
    print(json.dumps({
        "model": args.model, "batch": args.batch, "profile": args.profile, "runs": args.runs,
        "avg_s": avg, "images_per_sec": args.batch / avg,
        "threads": int(os.environ.get("OMP_NUM_THREADS", "0") or 0),
        "top1": int(out.reshape(args.batch, -1)[0].argmax()),
    }))


if __name__ == "__main__":
    main()
