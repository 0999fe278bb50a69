"""The committed tune table (spinnv2_amd/lib/mi355x.tune) against the
benchmark networks' layer shapes, on the CPU: every fp32 implicit-GEMM conv
and every INT8 conv of them has an entry under the key the runtime computes
(conv_f32.hip shape_key with the shared padded geometry, conv_i8.hip
tune_i8), so no process tunes them at prepare and fp32 results stay
bit-reproducible across processes (INT8 ResNet-50 in both INT8 modes); and
no conv entry is left over from a shape the networks no longer have."""

from __future__ import annotations

from pathlib import Path

import pytest

from spinnv2_amd import tune_table as T
from spinnv2_amd.spk import models

TABLE = Path(T.__file__).resolve().parent / "lib" / "mi355x.tune"


def _keys():
    f32, i8 = set(), set()
    graphs = [models.resnet(d, b) for d, b in ((101, 64), (101, 1), (18, 32), (18, 1))]
    graphs += [models.yolo_v10n(b) for b in (16, 1)]
    for g in graphs:
        for n in g.nodes:
            if n.op_type == "Conv" and n.attrs.get("group", 1) == 1 and not T._smallk(g, n):
                f32.add(T.f32_key(g, n))
    for b in (64, 1):
        g = models.resnet(50, b)
        i8.update(T.int8_key(g, n) for n in g.nodes if n.op_type == "Conv")
        # the INT8 configuration with int8 tensors between nodes: the same
        # layers under keys of their own (the key depends on shapes only)
        i8.update(T.int8_key(g, n, q8=True) for n in g.nodes if n.op_type == "Conv")
    return f32, i8


@pytest.fixture(scope="module")
def keys():
    return _keys()


def _table():
    return {line.split()[0] for line in TABLE.read_text().splitlines() if len(line.split()) == 3}


def test_every_benchmark_conv_has_an_entry(keys):
    f32, i8 = keys
    table = _table()
    assert not sorted(f32 - table), sorted(f32 - table)[:5]
    assert not sorted(i8 - table), sorted(i8 - table)[:5]


def test_no_stale_conv_entries(keys):
    f32, i8 = keys
    stale = sorted(k for k in _table() if k.startswith(("conv|", "i8|")) and k not in f32 | i8)
    assert not stale, stale[:5]


def test_shared_padded_geometry():
    """YOLOv10n: a conv output read by stride-1 and stride-2 padded 3x3 convs
    (a level's output: both head branches and the downsampling conv) gives
    them all the stride-1 geometry (82 x 82 at 80 x 80), so they can read one
    zero-padded copy; a stride-2 conv that is its input's only padded reader
    keeps its own (81 x 81); the RGB stem is not an implicit GEMM."""
    g = models.yolo_v10n(16)
    convs = [n for n in g.nodes if n.op_type == "Conv"]
    assert T._smallk(g, convs[0])
    down = [n for n in convs if g.shape(n.inputs[0])[2:] == [80, 80] and n.attrs.get("strides") == [2, 2]]
    shared = [n for n in down if any(r is not n and r.op_type == "Conv" and r.inputs[0] == n.inputs[0] and
                                     r.attrs.get("strides") == [1, 1] and r.attrs.get("pads", [0] * 4)[0] == 1
                                     for r in convs)]
    alone = [n for n in down if n not in shared]
    assert shared and alone
    assert all("|1,82,82|" in T.f32_key(g, n) for n in shared)
    assert all("|1,81,81|" in T.f32_key(g, n) for n in alone)
