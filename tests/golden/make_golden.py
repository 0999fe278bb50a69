"""Writes the golden fixtures in tests/golden/ from the reference SPINNV2 C runtime.

The reference runtime is compiled from its own sources under
/root/reference/runtime into oracle/_ref/libspkv2_ref.so (`make -C oracle
ref`); this script runs it on packages written by this repo's SPK writer with
the `cpu_ref` profile (every node on the reference kernels,
runtime/kernels/reference/*) -- or, for the `arm_*` cases, with the ARM
profiles whose conv kinds its optimized x86 kernels run -- and stores, per
case, the builder call, the profile, the inputs and the reference runtime's
output.  The fixtures are data only: the
tests re-create each package with the same builder call and compare the CPU
oracle (and, on the GPU box, the MI355X runtime) against the stored output.

    python tests/golden/make_golden.py          # rewrites tests/golden/*.npz

Needs /root/reference; the GPU box never runs this.
"""

from __future__ import annotations

import json
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent.parent
sys.path.insert(0, str(ROOT))

from oracle.ref_runtime import RefModel, available  # noqa: E402
from spinnv2_amd.spk import models, write_spk  # noqa: E402

# (fixture name, builder, kwargs, input distribution)
CASES: list[tuple[str, str, dict, str]] = []

# Conv shapes: the reference test suite's CONV_CASES flavour
# (tests/e2e/test_single_ops.py:72-80: kernel, stride, pad, group, dilation
# variations) at sizes the naive reference conv finishes quickly.
_CONV = [
    dict(n=1, cin=3, h=17, w=19, cout=8, k=3, stride=1, pad=1, act="Relu"),
    dict(n=2, cin=16, h=12, w=12, cout=32, k=1, stride=1, pad=0, act=None),
    dict(n=1, cin=3, h=32, w=32, cout=64, k=7, stride=2, pad=3, act="Relu"),
    dict(n=2, cin=64, h=14, w=14, cout=64, k=3, stride=1, pad=1, act="Relu", residual=True),
    dict(n=1, cin=32, h=15, w=15, cout=48, k=3, stride=2, pad=1, act="Silu"),
    dict(n=1, cin=8, h=16, w=16, cout=8, k=3, stride=1, pad=2, dilation=2, act=None, bias=False),
    dict(n=1, cin=16, h=10, w=10, cout=16, k=3, stride=1, pad=1, group=16, act="Relu"),
    dict(n=1, cin=16, h=10, w=10, cout=32, k=3, stride=1, pad=1, group=4, act=None),
    dict(n=1, cin=130, h=9, w=9, cout=70, k=1, stride=1, pad=0, act="Relu"),
    dict(n=3, cin=5, h=7, w=7, cout=3, k=3, stride=1, pad=1, act=None, residual=True),
    dict(n=1, cin=4, h=9, w=11, cout=6, k=3, stride=2, pad=0, act=None, pads=[0, 1, 1, 0]),
]
for i, kw in enumerate(_CONV):
    CASES.append((f"conv{i}", "single_conv", kw, "normal"))

_GEMM = [
    dict(rows=3, k=50, nout=20),
    dict(rows=5, k=64, nout=10, trans_b=1, alpha=0.5),
    dict(rows=1, k=2048, nout=100),
    dict(rows=7, k=33, nout=65, bias=False),
    dict(rows=4, k=33, nout=9, trans_b=1),
    dict(rows=3, k=7, nout=5, trans_b=1, alpha=2.0),
    dict(rows=2, k=3, nout=4, trans_b=1),
    # transA (reference mm/gemm.c:17-31: A read as [K][rows])
    dict(rows=5, k=33, nout=9, trans_a=1),
    dict(rows=4, k=20, nout=7, trans_a=1, trans_b=1, alpha=0.5),
]
for i, kw in enumerate(_GEMM):
    CASES.append((f"gemm{i}", "single_gemm", kw, "normal"))

_OPS = [
    ("MaxPool", [2, 8, 23, 23], dict(k=3, s=2, p=1)),
    ("MaxPool", [1, 4, 8, 8], dict(k=2, s=2, p=0)),
    ("Add", [2, 16, 9, 9], {}),
    ("Add", [2, 16, 9, 9], dict(b_shape=[1, 16, 1, 1])),
    ("Add", [1, 8, 5, 5], dict(relu=True)),
    ("Relu", [3, 7, 11], {}),
    ("Resize", [1, 4, 10, 12], dict(scale=2)),
    ("Softmax", [4, 1000], dict(axis=-1)),
    ("Softmax", [2, 16, 50], dict(axis=1)),
    ("ReduceMean", [2, 64, 7, 7], dict(axes=[2, 3])),
    ("ReduceMean", [2, 6, 5, 4], dict(axes=[1])),
    ("GlobalAveragePool", [2, 32, 7, 7], {}),
    ("AveragePool", [1, 4, 9, 9], dict(k=3, s=2, p=1)),
    ("Sigmoid", [2, 300], {}),
    ("Mul", [2, 8, 4, 4], dict(b_shape=[8, 1, 1])),
    ("Sub", [2, 3, 4], dict(b_shape=[4])),
    ("Div", [2, 3, 4], dict(b_shape=[3, 1])),
    # Mod (reference math/binary.c:25-26: C remainder of the truncated
    # operands); divisors kept at |b| >= 1 so the reference's int % never
    # divides by zero
    ("Mod", [2, 3, 4], dict(b_shape=[3, 1])),
]
for i, (op, shape, kw) in enumerate(_OPS):
    CASES.append((f"op{i}_{op}", "single_op", dict(op=op, shape=shape, **kw), "mod" if op == "Mod" else "normal"))

# Packages with the reference's optimized conv kinds, run by its x86 (AVX2)
# kernels: the cpu_arm_neon profile's Winograd F(4,3) (kind 9) with a fused
# residual, and the two kinds no reference profile selects but its runtime
# dispatches (kernels.c:75-77): Winograd F(2,3) (kind 7) and the 3x3/s2
# direct conv (kind 8); plus ResNet-18 at 64x64 under both ARM profiles.
# Their outputs carry the Winograd / AVX2 rounding, so they pin within the
# fp32 tolerance, not bit for bit.
CASES.append(("arm_f43_conv", "single_conv",
              dict(n=1, cin=32, h=12, w=12, cout=32, k=3, stride=1, pad=1, act="Relu", residual=True), "normal",
              "cpu_arm_neon"))
CASES.append(("arm_f23_conv", "single_conv", dict(n=2, cin=24, h=13, w=11, cout=40, k=3, stride=1, pad=1, act="Relu"),
              "normal", "cpu_arm_neon_exp"))
CASES.append(("arm_s2_conv", "single_conv", dict(n=2, cin=16, h=15, w=17, cout=24, k=3, stride=2, pad=1, act="Relu"),
              "normal", "cpu_arm_neon_exp"))
CASES.append(("arm_resnet18_64px", "resnet", dict(depth=18, batch=1, image=64, classes=10), "normal", "cpu_arm_neon"))
CASES.append(("arm_exp_resnet18_64px", "resnet", dict(depth=18, batch=1, image=64, classes=10), "normal",
              "cpu_arm_neon_exp"))

# Indexing / layout ops of the YOLO op set (reference tensor/*.c, shape/tile.c,
# shape/transpose.c).  Index tensors are constants; "ties" inputs are
# rounded to a coarse grid so TopK sees values tied across the k-th place.
_rng = np.random.default_rng(11)
_IDX = [
    ("Transpose", [2, 3, 4, 5], dict(perm=[0, 2, 3, 1])),
    ("Transpose", [6, 7], dict(perm=[1, 0])),
    ("Transpose", [1, 4, 2, 3, 5], dict(perm=[0, 3, 1, 4, 2])),
    ("Tile", [2, 3, 4], dict(reps=[1, 2, 3])),
    ("Split", [2, 10, 3, 3], dict(sizes=[2, 5, 3], axis=1)),
    ("Split", [4, 6], dict(sizes=[3, 3], axis=-1)),
    ("Slice", [3, 20, 4], dict(start=2, end=17, axis=1, step=3)),
    ("Slice", [5, 6], dict(start=-4, end=100, axis=0, step=1)),
    ("Gather", [5, 4, 3], dict(indices=[[4, 0], [-1, 2]], axis=0)),
    ("Gather", [2, 7, 3], dict(indices=[6, 1, -2, 0], axis=1)),
    ("GatherElements", [3, 5], dict(indices=_rng.integers(-5, 5, (3, 4)).tolist(), axis=1)),
    ("GatherElements", [4, 2, 3], dict(indices=_rng.integers(0, 4, (2, 2, 3)).tolist(), axis=0)),
    ("TopK", [3, 50], dict(k=7, axis=-1, largest=1)),
    ("TopK", [2, 40, 3], dict(k=10, axis=1, largest=0)),
    ("TopK", [1, 8400], dict(k=300, axis=-1, largest=1)),
    ("ReduceMax", [2, 6, 5, 4], dict(axes=[1, 3], keepdims=1)),
]
for i, (op, shape, kw) in enumerate(_IDX):
    CASES.append((f"idx{i}_{op}", "index_op", dict(op=op, shape=shape, **kw), "normal"))
CASES.append(("idx_topk_ties", "index_op", dict(op="TopK", shape=[2, 200], k=30, axis=-1, largest=1), "ties"))
CASES.append(("idx_topk_ties_small", "index_op", dict(op="TopK", shape=[3, 64], k=9, axis=-1, largest=0), "ties"))

# Batched MatMul (reference kernels/reference/mm/matmul.c): plain 2-D,
# batched, leading-dim broadcasting both ways, a constant B, odd sizes that
# leave partial 64x64 tiles, and the two PSA attention products of the
# YOLOv10n-style graph at 320 (100 positions, 2 heads).
_MATMUL = [
    dict(a_shape=[5, 7], b_shape=[7, 3]),
    dict(a_shape=[2, 3, 8, 16], b_shape=[2, 3, 16, 5]),
    dict(a_shape=[2, 1, 4, 6], b_shape=[3, 6, 5]),
    dict(a_shape=[3, 70, 33], b_shape=[33, 65]),
    dict(a_shape=[4, 33, 17], b_shape=[17, 9], const_b=True),
    dict(a_shape=[1, 2, 100, 32], b_shape=[1, 2, 32, 100]),
    dict(a_shape=[1, 2, 64, 100], b_shape=[1, 2, 100, 100]),
]
for i, kw in enumerate(_MATMUL):
    CASES.append((f"matmul{i}", "matmul_op", kw, "normal"))

# End to end: the LeNet config on U[0,1) input, and a
# ResNet-18 at 32x32 (every ResNet node kind: stem, pools, basic blocks with
# projections, ReduceMean, Gemm).
CASES.append(("lenet", "lenet", {}, "uniform"))
CASES.append(("resnet18_32px", "resnet", dict(depth=18, batch=2, image=32, classes=10), "normal"))
CASES.append(("resnet50_32px", "resnet", dict(depth=50, batch=1, image=32, classes=10), "normal"))
# the YOLOv10n-style detector at 160x160: 525 anchors, TopK(300)
CASES.append(("yolov10n_160", "yolo_v10n", dict(image=160), "uniform"))


def build_graph(builder: str, kw: dict):
    kw = dict(kw)
    if builder in ("single_op", "index_op"):
        op = kw.pop("op")
        shape = kw.pop("shape")
        return getattr(models, builder)(op, shape, **kw)
    return getattr(models, builder)(**kw)


def case_inputs(g, dist: str, seed: int = 42) -> list[np.ndarray]:
    if dist == "ties":  # values on a coarse grid: many exact ties
        return [np.round(models.make_input(g.tensors[t].shape, seed + i, "normal") * 2).astype(np.float32) / 2
                for i, t in enumerate(g.inputs)]
    if dist == "mod":  # dividend N(0, 20^2); divisor of magnitude in [1, 7.9), either sign
        a = models.make_input(g.tensors[g.inputs[0]].shape, seed, "normal") * np.float32(20)
        u = models.make_input(g.tensors[g.inputs[1]].shape, seed + 1, "uniform")
        b = (np.floor(u * 7) + 1 + 0.9 * np.abs(np.sin(u * 97))) * np.where(u < 0.5, -1, 1)
        return [a.astype(np.float32), b.astype(np.float32)]
    return [models.make_input(g.tensors[t].shape, seed + i, dist) for i, t in enumerate(g.inputs)]


def main() -> None:
    if not available():
        sys.exit("oracle/_ref/libspkv2_ref.so is not built: make -C oracle ref (needs /root/reference)")
    only = set(sys.argv[1:])
    for case in CASES:
        name, builder, kw, dist = case[:4]
        profile = case[4] if len(case) > 4 else "cpu_ref"
        if only and name not in only:
            continue
        g = build_graph(builder, kw)
        blob = write_spk(g, profile)
        xs = case_inputs(g, dist)
        ref = RefModel(blob)
        ys = [ref.run(*xs, output=o) for o in range(len(g.outputs))]
        ref.close()
        y = ys[0]
        if profile != "cpu_ref" and name != "arm_s2_conv":
            # a Winograd kernel, not the naive reference conv, ran: the bits
            # differ (the 3x3/s2 direct kernel sums in the naive conv's order
            # and matches it bit for bit)
            naive = RefModel(write_spk(build_graph(builder, kw), "cpu_ref"))
            y0 = naive.run(*xs)
            naive.close()
            assert not np.array_equal(y.view(np.uint32), y0.view(np.uint32)), name
        meta = {"builder": builder, "kwargs": kw, "dist": dist, "seed": 42, "profile": profile,
                "source": "reference runtime (runtime/core + runtime/kernels/reference"
                          + (" + runtime/kernels/optimized, x86 AVX2" if profile != "cpu_ref" else "")
                          + ") built by oracle/Makefile"}
        arrays = {f"x{i}": x for i, x in enumerate(xs)}
        arrays.update({f"y{o}": v for o, v in enumerate(ys) if o > 0})
        np.savez_compressed(HERE / f"{name}.npz", meta=np.frombuffer(json.dumps(meta).encode(), dtype=np.uint8),
                            y=y, **arrays)
        print(f"{name:24s} inputs {[list(x.shape) for x in xs]} -> {y.size} values")


if __name__ == "__main__":
    main()
