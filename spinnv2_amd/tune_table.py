"""Regenerates spinnv2_amd/lib/mi355x.tune, the tile / split-K choices the
runtime uses for the benchmark networks' layer shapes (read beside the
library, so every process picks the same configuration for them and fp32
results are bit-reproducible across processes).

Needs the GPU: every conv and Gemm of each network is prepared once with
the built-in table ignored (SPKV2_TUNE_TABLE=0), so the prepare-time tuner
times its candidates and appends its choice to the output file
(SPKV2_TUNE_DB); the file is then sorted and de-duplicated.

    python -m spinnv2_amd.tune_table [out.tune] [--retune-int8]

INT8 entries (keys starting `i8|`) already in the committed table are kept
unless --retune-int8 is given: the INT8 tuner times each layer alone with an
fp32 epilogue, while in the network most int8 convs hand int8 to the next
conv instead, and on ResNet-50 b=64 a regenerated set of INT8 choices ran the
network at 1.97 ms per step against 1.80 for the kept one.
"""

from __future__ import annotations

import os
import sys
from pathlib import Path

DEFAULT_OUT = Path(__file__).resolve().parent / "lib" / "mi355x.tune"


def networks():
    """(label, graph, quant params) of every benchmark configuration."""
    from .spk import models
    from .spk.quantize import calibrate_activation_scales, quantize_conv_weights

    for depth, batch in ((101, 64), (101, 1), (18, 32), (18, 1)):
        yield f"resnet{depth} b={batch}", models.resnet(depth, batch), None
    g1 = models.resnet(50, 1)
    samples = [models.make_input(g1.tensors[g1.inputs[0]].shape, 1000 + i) for i in range(16)]
    act = calibrate_activation_scales(g1, samples)
    for batch in (64, 1):
        g = models.resnet(50, batch)
        yield f"int8 resnet50 b={batch}", g, quantize_conv_weights(g) + act
    for batch in (16, 1):
        yield f"yolov10n b={batch}", models.yolo_v10n(batch), None


def main() -> None:
    args = [a for a in sys.argv[1:] if not a.startswith("--")]
    retune_int8 = "--retune-int8" in sys.argv[1:]
    out = Path(args[0]) if args else DEFAULT_OUT
    kept = {}
    if not retune_int8 and DEFAULT_OUT.exists():
        for line in DEFAULT_OUT.read_text().splitlines():
            if line.startswith("i8|") and len(line.split()) == 3:
                kept[line.split()[0]] = line
    tmp = out.with_suffix(".partial")
    tmp.unlink(missing_ok=True)
    os.environ["SPKV2_TUNE_TABLE"] = "0"
    os.environ["SPKV2_TUNE_DB"] = str(tmp)
    for k in ("SPKV2_CONV_CFG", "SPKV2_CONV_SPLITK", "SPKV2_CONV_HYBRID", "SPKV2_CONV_TUNE", "SPKV2_I8_CFG",
              "SPKV2_I8_SPLITK"):
        os.environ.pop(k, None)
    from .runtime import Model, load_library
    from .spk import write_spk

    lib = load_library()
    for label, g, qp in networks():
        with Model(write_spk(g, "mi355x", quant_params=qp), lib=lib):
            pass
        print(f"tuned {label}", flush=True)
    lines = {}
    for line in tmp.read_text().splitlines():
        parts = line.split()
        if len(parts) == 3:
            lines[parts[0]] = line
    lines.update(kept)
    out.write_text("".join(lines[k] + "\n" for k in sorted(lines)))
    tmp.unlink()
    print(f"{len(lines)} layer shapes -> {out}")


if __name__ == "__main__":
    main()
