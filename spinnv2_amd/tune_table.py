"""Regenerates spinnv2_amd/lib/mi355x.tune, the tile / split-K choices the
runtime uses for the benchmark networks' layer shapes (read beside the
library, so every process picks the same configuration for them and fp32
results are bit-reproducible across processes).

Needs the GPU: every conv and Gemm of each network is prepared once with
the built-in table ignored (SPKV2_TUNE_TABLE=0), so the prepare-time tuner
times its candidates and appends its choice to the output file
(SPKV2_TUNE_DB); the file is then sorted and de-duplicated.

    python -m spinnv2_amd.tune_table [out.tune] [--retune-int8 | --missing] [--no-int8]
    python -m spinnv2_amd.tune_table --int8-network [--b1 | --splitk] [table.tune]
    python -m spinnv2_amd.tune_table --q8-network [--b1 | --splitk] [table.tune]
    python -m spinnv2_amd.tune_table --f32-network [--yolo] [--b1] [--thin | --rows96 | --skinny] [table.tune]

With --missing every entry of the committed table is kept and only layer
shapes it lacks are tuned (the table stays in force, so the tuner runs for
those alone); --no-int8 leaves the INT8 networks out.  INT8 entries (keys starting `i8|`) already in the committed
table are kept unless --retune-int8 is given: the INT8 tuner times each layer alone with an
fp32 epilogue, while in the network most int8 convs hand int8 to the next
conv instead, and on ResNet-50 b=64 a regenerated set of INT8 choices ran the
network at 1.97 ms per step against 1.80 for the kept one.

--int8-network chooses the batch-64 INT8 entries inside the network instead:
one process per tile configuration (the table and tune DB are read once per
process) maps every INT8 layer shape of ResNet-50 b=64 to that configuration
through a private tune DB, and times every conv node of the network (HIP
events per node, 3 warmup + 10 runs); a shape whose layout does not allow
the configuration falls back to the tuner, which appends its own choice to
the DB, so those shapes are left out of that configuration's figures.  A
shape's entry changes when another configuration's summed node time over
its nodes beats the current one by more than 2%.  --f32-network does the
same for ResNet-101 b=64 (with --yolo YOLOv10n b=16, with --b1 batch 1)
over the fp32 tile configurations and schedules (F32_SWEEP, F32_SWEEP_B1),
or with --thin / --rows96 / --skinny over the thin, the 96-row or the skinny
and row-window tiles alone (F32_THIN, F32_ROWS96, F32_SKINNY).  --q8-network does it for the INT8 configuration with int8
tensors between nodes (ResNet-50, keys ending in |q8) over every int8 tile
configuration, the persistent ones included.
"""

from __future__ import annotations

import os
import sys
from pathlib import Path

DEFAULT_OUT = Path(__file__).resolve().parent / "lib" / "mi355x.tune"


def networks(int8: bool = True):
    """(label, graph, quant params) of every benchmark configuration (without
    the INT8 ones when int8 is false)."""
    from .spk import models
    from .spk.quantize import calibrate_activation_scales, quantize_conv_weights

    for depth, batch in ((101, 64), (101, 1), (18, 32), (18, 1)):
        yield f"resnet{depth} b={batch}", models.resnet(depth, batch), None
    if int8:
        g1 = models.resnet(50, 1)
        samples = [models.make_input(g1.tensors[g1.inputs[0]].shape, 1000 + i) for i in range(16)]
        act = calibrate_activation_scales(g1, samples)
        for batch in (64, 1):
            g = models.resnet(50, batch)
            yield f"int8 resnet50 b={batch}", g, quantize_conv_weights(g) + act
    for batch in (16, 1):
        yield f"yolov10n b={batch}", models.yolo_v10n(batch), None
    if int8:
        for batch in (64, 1):
            yield f"int8 configuration resnet50 b={batch}", *q8_resnet50(batch)


def main() -> None:
    args = [a for a in sys.argv[1:] if not a.startswith("--")]
    retune_int8 = "--retune-int8" in sys.argv[1:]
    missing = "--missing" in sys.argv[1:]
    out = Path(args[0]) if args else DEFAULT_OUT
    kept = {}
    if not retune_int8 and DEFAULT_OUT.exists():
        for line in DEFAULT_OUT.read_text().splitlines():
            if (missing or line.startswith("i8|")) and len(line.split()) == 3:
                kept[line.split()[0]] = line
    tmp = out.with_suffix(".partial")
    tmp.unlink(missing_ok=True)
    # --missing: the table stays in force, so only shapes it lacks are tuned
    os.environ["SPKV2_TUNE_TABLE"] = "1" if missing else "0"
    os.environ["SPKV2_TUNE_DB"] = str(tmp)
    for k in ("SPKV2_CONV_CFG", "SPKV2_CONV_SPLITK", "SPKV2_CONV_HYBRID", "SPKV2_CONV_TUNE", "SPKV2_I8_CFG",
              "SPKV2_I8_SPLITK"):
        os.environ.pop(k, None)
    from .runtime import Model, load_library
    from .spk import write_spk

    lib = load_library()
    for label, g, qp in networks(int8="--no-int8" not in sys.argv[1:]):
        blob = qp if isinstance(qp, bytes) else write_spk(g, "mi355x", quant_params=qp)
        with Model(blob, lib=lib):
            pass
        print(f"tuned {label}", flush=True)
    lines = {}
    for line in (tmp.read_text() if tmp.exists() else "").splitlines():
        parts = line.split()
        if len(parts) == 3:
            lines[parts[0]] = line
    lines.update(kept)
    out.write_text("".join(lines[k] + "\n" for k in sorted(lines)))
    tmp.unlink(missing_ok=True)
    print(f"{len(lines)} layer shapes -> {out}")


def int8_key(g, n, q8: bool = False) -> str:
    """The INT8 tuner's key of a conv node (conv_i8.hip, tune_i8); q8: the
    INT8 configuration with int8 tensors between nodes."""
    x, w, y = g.shape(n.inputs[0]), g.tensors[n.inputs[1]].shape, g.shape(n.outputs[0])
    st, dl = n.attrs.get("strides", [1, 1]), n.attrs.get("dilations", [1, 1])
    return (f"i8|{x[0]},{x[1]},{x[2]},{x[3]}|{w[0]},{w[2]},{w[3]},{y[2]},{y[3]},{st[0]},{st[1]},{dl[0]},{dl[1]}|"
            f"{1 if len(n.inputs) > 2 else 0},{1 if len(n.inputs) > 3 else 0},{_act(n)}" + ("|q8" if q8 else ""))


def q8_resnet50(batch: int):
    """INT8 ResNet-50 224x224 in the INT8 configuration with int8 tensors
    between nodes, calibrated as bench.py does (16 seeded single-image
    batches through the batch-1 fp32 graph): (graph, package)."""
    from .spk import models, write_spk
    from .spk.quantize import quantize_int8_activations

    cal = models.resnet(50, 1)
    samples = [models.make_input(cal.tensors[cal.inputs[0]].shape, 1000 + i) for i in range(16)]
    g = models.resnet(50, batch)
    return g, write_spk(g, "mi355x", quant_params=quantize_int8_activations(g, samples, calibrate_on=cal))


def _padded_extent(g, n):
    """(padded, Hp, Wp) of a conv node's own zero-padded input (conv_f32.hip,
    padded_extent)."""
    _, _, H, W = g.shape(n.inputs[0])
    _, _, KH, KW = g.tensors[n.inputs[1]].shape
    OH, OW = g.shape(n.outputs[0])[2:]
    sh, sw = n.attrs.get("strides", [1, 1])
    dh, dw = n.attrs.get("dilations", [1, 1])
    ph, pw = n.attrs.get("pads", [0, 0, 0, 0])[:2]
    hspan, wspan = (OH - 1) * sh + (KH - 1) * dh + 1, (OW - 1) * sw + (KW - 1) * dw + 1
    padded = ph > 0 or pw > 0 or hspan - ph > H or wspan - pw > W
    return padded, max(H + ph, hspan), max(W + pw, wspan)


def _smallk(g, n) -> bool:
    """Whether the small-gather stem kernel takes the conv (conv_f32.hip, smallk_fits)."""
    C = g.shape(n.inputs[0])[1]
    M, _, KH, KW = g.tensors[n.inputs[1]].shape
    return n.attrs.get("group", 1) == 1 and C <= 4 and C * KH * KW <= 64 and M <= 64


def f32_key(g, n) -> str:
    """The fp32 tuner's key of a group-1 conv node (conv_f32.hip, shape_key
    and plan_igemm_f32's padded-input geometry: the largest any padded conv
    reader of the same conv output needs, shared_pad_extent)."""
    N, C, H, W = g.shape(n.inputs[0])
    M, _, KH, KW = g.tensors[n.inputs[1]].shape
    OH, OW = g.shape(n.outputs[0])[2:]
    sh, sw = n.attrs.get("strides", [1, 1])
    dh, dw = n.attrs.get("dilations", [1, 1])
    pads = n.attrs.get("pads", [0, 0, 0, 0])[:2]
    padded, Hp, Wp = _padded_extent(g, n)
    if padded:
        prod = [p for p in g.nodes if p.id < n.id and n.inputs[0] in p.outputs]
        if prod and prod[-1].op_type == "Conv":
            for r in g.nodes:
                if (r.op_type != "Conv" or r.inputs[0] != n.inputs[0] or r.attrs.get("group", 1) != 1 or _smallk(g, r)
                        or r.attrs.get("pads", [0, 0, 0, 0])[:2] != pads):
                    continue
                rp, rh, rw = _padded_extent(g, r)
                if rp:
                    Hp, Wp = max(Hp, rh), max(Wp, rw)
    else:
        Hp, Wp = H, W
    return (f"conv|{N},{C},{H},{W}|{M},{KH},{KW},{OH},{OW},{sh},{sw},{dh}|{dw},{Hp},{Wp}|{C * Hp * Wp},"
            f"{1 if len(n.inputs) > 2 else 0},{1 if len(n.inputs) > 3 else 0},{_act(n)}")


def _act(n) -> int:
    from .spk import format as F

    return int(F.ACTIVATION[n.attrs.get("fused_activation")])


def _sweep_child(blob: str, cand: str, out: str) -> None:
    """One candidate of an in-network sweep: every key in blob + '.keys' set
    to `cand` ("cfg split", or "table": the committed table as is) through a
    private tune DB; writes each conv node's time and the keys that fell back
    to the tuner (their layout does not allow the candidate)."""
    import json

    import numpy as np

    keys = json.loads(Path(blob + ".keys").read_text())
    if cand != "table":
        db = out + ".tune"
        Path(db).write_text("".join(f"{k} {cand}\n" for k in keys))
        os.environ["SPKV2_TUNE_TABLE"] = "0"
        os.environ["SPKV2_TUNE_DB"] = db
    from .runtime import DeviceBuffer, Model, load_library

    meta = json.loads(Path(blob + ".ids").read_text())
    lib = load_library()
    m = Model(Path(blob).read_bytes(), lib=lib)
    from .spk import models

    x = models.make_input(meta["input"])
    buf = DeviceBuffer(x.nbytes, lib)
    buf.upload(np.ascontiguousarray(x))
    m.bind_input(0, buf)
    m.set_profiling(True)
    for _ in range(3):
        m.run()
    m.reset_node_times()
    for _ in range(10):
        m.run()
    lib.spkv2_device_synchronize()
    times = {}
    for i in meta["ids"]:
        ms, c = m.node_time(i)
        times[i] = ms / max(c, 1) * 1e3
    m.close()
    buf.free()
    fell_back = set()
    if cand != "table":
        for line in Path(out + ".tune").read_text().splitlines()[len(keys):]:
            if line.split():
                fell_back.add(line.split()[0])
    Path(out).write_text(json.dumps({"times": times, "fell_back": sorted(fell_back)}))


def network_sweep(g, blob: bytes, keys: dict, candidates, table: Path, label: str, open_ended: bool = False) -> None:
    """Times every candidate (cfg, split) on the network in a process of its
    own and rewrites the table entries of `keys` (node id -> key) whose
    summed node time some candidate beats by more than 2%.  With open_ended
    (configuration indices counted up without a known end) a candidate no
    key takes ends the sweep; otherwise it is only skipped."""
    import json
    import subprocess
    import tempfile

    current = {}
    for line in table.read_text().splitlines():
        p = line.split()
        if len(p) == 3:
            current[p[0]] = (int(p[1]), int(p[2]))
    allkeys = sorted(set(keys.values()))
    runs = {}
    with tempfile.TemporaryDirectory() as d:
        bp = os.path.join(d, "net.spk")
        Path(bp).write_bytes(blob)
        Path(bp + ".ids").write_text(json.dumps({"ids": sorted(keys), "input": list(g.shape(g.inputs[0]))}))
        Path(bp + ".keys").write_text(json.dumps(allkeys))
        for cand in ["table", *[f"{c} {s}" for c, s in candidates]]:
            out = os.path.join(d, "cand.json")
            r = subprocess.run([sys.executable, "-m", "spinnv2_amd.tune_table", "--sweep-child", bp, cand, out],
                               capture_output=True, text=True)
            if r.returncode != 0:
                raise RuntimeError(f"{label} sweep, candidate {cand}:\n{r.stderr[-2000:]}")
            res = json.loads(Path(out).read_text())
            if cand != "table" and set(res["fell_back"]) >= set(allkeys):
                if open_ended:
                    break
                continue
            runs[cand] = res
            print(f"{label}: candidate {cand} timed", flush=True)
    base = runs.pop("table")
    changed = {}
    for key in allkeys:
        nodes = [str(i) for i, k in keys.items() if k == key]
        now = sum(base["times"][i] for i in nodes)
        best, pick = now, None
        for cand, r in runs.items():
            if key in r["fell_back"]:
                continue
            t = sum(r["times"][i] for i in nodes)
            if t < best:
                best, pick = t, cand
        if key not in current:
            # not in the table yet (the live tuner ran for it): the best
            # explicit candidate, so the choice becomes reproducible
            best, pick = 1e300, None
            for cand, r in runs.items():
                if key in r["fell_back"]:
                    continue
                t = sum(r["times"][i] for i in nodes)
                if t < best:
                    best, pick = t, cand
            if pick:
                changed[key] = pick
                print(f"{key}: new -> {pick} ({now:.1f} us with the live tuner, {best:.1f} us)")
            continue
        if pick and tuple(map(int, pick.split())) != current.get(key) and best < 0.98 * now:
            changed[key] = pick
            print(f"{key}: {current.get(key)} -> {pick} ({now:.1f} -> {best:.1f} us over {len(nodes)} nodes)")
    lines = []
    for line in table.read_text().splitlines():
        p = line.split()
        lines.append(f"{p[0]} {changed[p[0]]}" if p and p[0] in changed else line)
    lines += [f"{k} {v}" for k, v in changed.items() if k not in current]
    lines = sorted(set(lines), key=lambda l: l.split()[0] if l.split() else "")
    table.write_text("".join(l + "\n" for l in lines))
    print(f"{label}: {len(changed)} entries changed -> {table}")


# conv_i8.hip's tile configurations (kI8Cfgs): how many, and those that
# take split-K (the persistent ones, 23-30, 35 and 36, take whole tiles only)
I8_CONFIGS = 37
I8_SPLITTABLE = [*range(23), 31, 32, 33, 34]


def int8_network(table: Path, batch: int = 64) -> None:
    from .spk import models, write_spk
    from .spk.quantize import calibrate_activation_scales, quantize_conv_weights

    g1 = models.resnet(50, 1)
    samples = [models.make_input(g1.tensors[g1.inputs[0]].shape, 1000 + i) for i in range(16)]
    act = calibrate_activation_scales(g1, samples)
    g = models.resnet(50, batch)
    blob = write_spk(g, "mi355x", quant_params=quantize_conv_weights(g) + act)
    keys = {n.id: int8_key(g, n) for n in g.nodes if n.op_type == "Conv"}
    if batch == 1:  # every configuration with split-K too
        network_sweep(g, blob, keys, [(c, s) for c in I8_SPLITTABLE for s in (1, 2, 3, 4, 6, 8, 12, 16)], table,
                      "int8 resnet50 b=1")
    elif "--splitk" in sys.argv[1:]:  # the configurations with split-K 2, 3, 4
        network_sweep(g, blob, keys, [(c, s) for c in I8_SPLITTABLE for s in (2, 3, 4)], table, "int8 resnet50 b=64")
    else:
        network_sweep(g, blob, keys, [(c, 1) for c in range(64)], table, "int8 resnet50 b=64", open_ended=True)


def q8_network(table: Path, batch: int = 64) -> None:
    """In-network sweep of the INT8 configuration's layers (keys ending in
    |q8): every int8 tile configuration, whole tiles (and at batch 1 with
    split-K)."""
    g, blob = q8_resnet50(batch)
    keys = {n.id: int8_key(g, n, q8=True) for n in g.nodes if n.op_type == "Conv"}
    if batch == 1:
        cands = [(c, s) for c in range(I8_CONFIGS) for s in (1, 2, 3, 4, 6, 8, 12, 16)
                 if s == 1 or c in I8_SPLITTABLE]
    else:
        cands = [(c, 1) for c in range(I8_CONFIGS)] + ([(c, s) for c in I8_SPLITTABLE for s in (2, 3, 4)]
                                                       if "--splitk" in sys.argv[1:] else [])
    network_sweep(g, blob, keys, cands, table, f"int8 configuration resnet50 b={batch}")


# fp32 candidates: every configuration but the skinny ones (batch-1 tiles)
# whole-tile, and the hybrid schedules the tuner picks for ResNet-101 b=64
# (1000 + slices per remaining tile) on the 64-row ones and on the 128 x 64
# tiles with the waves along M
F32_SWEEP = [(c, 1) for c in (0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 14, 15, 16, 25, 26)] + \
            [(c, s) for c in (2, 6, 7, 25) for s in (1004, 1008, 1016)] + [(6, 3), (26, 1008)]


# batch 1: every configuration but the thin and 96-row ones, whole tiles and
# split-K (the skinny and row-window ones split k over their waves instead)
F32_SWEEP_B1 = [(c, s) for c in (*range(17), 21, 22, 23, 24) for s in (1, 2, 3, 4, 6, 8, 12, 16)
                if s == 1 or c not in (12, 13, 21, 22, 23, 24)]

# the thin tiles alone (16 and 32 rows by 256 columns, whole tiles), against
# the table as it is
F32_THIN = [(17, 1), (18, 1)]

# the 96-row tiles (whole tiles and hybrid schedules), against the table as it is
F32_ROWS96 = [(c, s) for c in (19, 20) for s in (1, 1004, 1008)]

# the skinny and row-window tiles (4, 8 and 16 waves), against the table as it is
F32_SKINNY = [(c, 1) for c in (12, 13, 23, 21, 22, 24)]


def f32_network(table: Path, net: str = "resnet101", thin: bool = False, rows96: bool = False,
                skinny: bool = False) -> None:
    from .spk import models, write_spk

    g = {"yolo": lambda: models.yolo_v10n(16), "yolo_b1": lambda: models.yolo_v10n(1),
         "resnet101_b1": lambda: models.resnet(101, 1)}.get(net, lambda: models.resnet(101, 64))()
    blob = write_spk(g, "mi355x")
    keys = {n.id: f32_key(g, n) for n in g.nodes
            if n.op_type == "Conv" and n.attrs.get("group", 1) == 1 and not _smallk(g, n)}
    cands = F32_SKINNY if skinny else F32_ROWS96 if rows96 else F32_THIN if thin else \
        F32_SWEEP_B1 if net in ("resnet101_b1", "yolo_b1") else \
        F32_SWEEP + ([(c, s) for c in (14, 15, 16) for s in (1004, 1008, 1016)] if net == "yolo" else [])
    network_sweep(g, blob, keys, cands, table, {"yolo": "yolov10n b=16", "yolo_b1": "yolov10n b=1",
                                                "resnet101_b1": "resnet101 b=1"}.get(net, "resnet101 b=64"))


if __name__ == "__main__":
    if len(sys.argv) == 5 and sys.argv[1] == "--sweep-child":
        _sweep_child(sys.argv[2], sys.argv[3], sys.argv[4])
    elif any(f in sys.argv[1:] for f in ("--int8-network", "--f32-network", "--q8-network")):
        rest = [a for a in sys.argv[1:] if not a.startswith("--")]
        table = Path(rest[0]) if rest else DEFAULT_OUT
        if "--q8-network" in sys.argv[1:]:
            q8_network(table, 1 if "--b1" in sys.argv[1:] else 64)
        elif "--int8-network" in sys.argv[1:]:
            int8_network(table, 1 if "--b1" in sys.argv[1:] else 64)
        else:
            yolo, b1 = "--yolo" in sys.argv[1:], "--b1" in sys.argv[1:]
            f32_network(table, ("yolo_b1" if b1 else "yolo") if yolo else "resnet101_b1" if b1 else "resnet101",
                        thin="--thin" in sys.argv[1:], rows96="--rows96" in sys.argv[1:],
                        skinny="--skinny" in sys.argv[1:])
    else:
        main()
