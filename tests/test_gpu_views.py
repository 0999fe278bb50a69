"""GPU: Concat and Split along channels without copies (channel-slice
views, spinnv2_amd/csrc/kernels/views.cpp).

The producers of a Concat's inputs write them into the Concat's buffer and
their readers read them there; every output must equal the copying path bit
for bit (the same arithmetic on the same values) and the oracle within the
fp32 tolerance.  Reference semantics: runtime/kernels/reference/tensor/
concat.c and split.c (copies).
"""

from __future__ import annotations

import numpy as np
import pytest

from spinnv2_amd.spk import models, write_spk
from spinnv2_amd.spk.graph import Graph
from spinnv2_amd.spk.passes import run_default_pipeline

from .helpers import FP32_TOL, rng_inputs, run_oracle, tnorm_err

pytestmark = pytest.mark.gpu


def _c2f_graph(batch: int, c_in: int = 16, hw: int = 20, widths=(16, 64)) -> Graph:
    """Two C2f blocks (Conv 1x1 -> Split -> bottlenecks -> Concat -> Conv
    1x1), the first with shortcut Adds (by default 8-channel halves: 3x3
    convs on implicit padding), the second without shortcuts (32-channel
    halves: 3x3 convs on a padded copy), then a Concat of two convs (both
    inputs written in place) and a graph output that is not a view."""
    p = models.Params(11)
    g = Graph("c2f_views")
    x = g.input("x", [batch, c_in, hw, hw])
    h = models._c2f(g, p, x, widths[0], 2, shortcut=True)
    h = models._c2f(g, p, h, widths[1], 1, shortcut=False)
    a = models._cbs(g, p, h, 24, 1)
    b = models._cbs(g, p, h, 40, 3)
    y = models._cbs(g, p, g.concat([a, b], axis=1), 32, 1)
    g.mark_output(y)
    run_default_pipeline(g)
    return g


def _run(blob: bytes, xs, nodes: int, *, graph: bool = False, fault=None):
    from spinnv2_amd.runtime import Model

    with Model(blob) as m:
        if fault is not None:
            m.set_fault_event(fault)
        m.set_graph_mode(graph)
        outs = []
        for _ in range(3 if graph else 1):
            for i, x in enumerate(xs):
                m.set_input(i, x)
            m.run()
            outs.append(m.get_output(0))
        names = [m.kernel_name(i) for i in range(nodes)]
    for o in outs[1:]:
        np.testing.assert_array_equal(o, outs[0])
    return outs[0], names


@pytest.mark.parametrize("split", ["auto", "3"])
def test_c2f_views_bit_identical_to_copies(gpu, monkeypatch, split):
    """Views on (Splits and Concats skip their copies) equal views off bit
    for bit, and the oracle within tolerance; forced split-K (the split-K
    epilogue writes through the view) as well."""
    if split != "auto":
        monkeypatch.setenv("SPKV2_CONV_SPLITK", split)
    g = _c2f_graph(batch=2)
    blob = write_spk(g, "mi355x")
    xs = rng_inputs(g)
    print(f"[views] c2f batch 2 split={split}", flush=True)
    monkeypatch.setenv("SPKV2_CONCAT_VIEWS", "1")
    on, names_on = _run(blob, xs, len(g.nodes))
    monkeypatch.setenv("SPKV2_CONCAT_VIEWS", "0")
    off, names_off = _run(blob, xs, len(g.nodes))
    np.testing.assert_array_equal(on.view(np.uint32), off.view(np.uint32))
    assert names_on.count("split_views") == 2, names_on
    assert names_on.count("concat_views") == 3, names_on
    assert "binary_img4" in names_on
    assert "split_views" not in names_off and "concat_views" not in names_off
    want = run_oracle(blob, xs)[0]
    assert tnorm_err(on, want) <= FP32_TOL


@pytest.mark.parametrize("cfg,kind", [("12", "skinny"), ("21", "window"), ("24", "window")],
                         ids=["skinny4", "window4", "window16"])
def test_c2f_views_skinny_kernel(gpu, monkeypatch, cfg, kind):
    """The skinny 16x16 kernel and its row-window form (layers of 64-channel
    multiples) reading and writing through views and padded-input handoffs:
    every conv that can take it is forced onto it."""
    monkeypatch.setenv("SPKV2_CONV_CFG", cfg)
    g = _c2f_graph(batch=2, c_in=64, hw=12, widths=(128, 128))
    blob = write_spk(g, "mi355x")
    xs = rng_inputs(g)
    on, names = _run(blob, xs, len(g.nodes))
    monkeypatch.setenv("SPKV2_CONCAT_VIEWS", "0")
    off, _ = _run(blob, xs, len(g.nodes))
    np.testing.assert_array_equal(on.view(np.uint32), off.view(np.uint32))
    assert any(kind in n for n in names), names
    assert "concat_views" in names


def test_c2f_views_thin_kernel(gpu, monkeypatch):
    """The thin kernel (no LDS, one wave per 64 columns) reading and writing
    through views and handoffs: every conv that can take it is forced onto
    it; views on equal views off bit for bit, and the oracle within
    tolerance."""
    monkeypatch.setenv("SPKV2_CONV_CFG", "18")
    g = _c2f_graph(batch=2, c_in=16, hw=20, widths=(32, 64))
    blob = write_spk(g, "mi355x")
    xs = rng_inputs(g)
    on, names = _run(blob, xs, len(g.nodes))
    monkeypatch.setenv("SPKV2_CONCAT_VIEWS", "0")
    off, _ = _run(blob, xs, len(g.nodes))
    np.testing.assert_array_equal(on.view(np.uint32), off.view(np.uint32))
    assert sum("conv_thin_f32" in n for n in names) >= 6, names
    assert "concat_views" in names
    assert tnorm_err(on, run_oracle(blob, xs)[0]) <= FP32_TOL


def test_c2f_views_graph_mode_and_fault_path(gpu):
    """HIP-graph replays with the views equal eager; with a fault event
    armed (an injection that never fires) the views are off and every
    Split / Concat copies, with the same result."""
    from spinnv2_amd.runtime import FaultEvent

    g = _c2f_graph(batch=3)
    blob = write_spk(g, "mi355x")
    xs = rng_inputs(g)
    eager, names = _run(blob, xs, len(g.nodes))
    assert "concat_views" in names
    replay, _ = _run(blob, xs, len(g.nodes), graph=True)
    np.testing.assert_array_equal(replay, eager)
    ev = FaultEvent(node_id=0, tensor_id=g.nodes[0].outputs[0], element_index=0, bit_index=0,
                    invocation_index=1000, seed=0, enabled=1)
    faulted, names_f = _run(blob, xs, len(g.nodes), fault=ev)
    np.testing.assert_array_equal(faulted, eager)
    assert "concat_views" not in names_f and "split_views" not in names_f


# batch -> (Splits, Concats) without copies: the eight C2f blocks' Splits;
# at batch 1 only the Concats whose every input is placed (the C2f ones,
# SPPF's -- its stride-1 MaxPools read and write the buffer -- and the PAN
# Concat whose other input is a conv's: the 2x Resize writes its upsampled
# input in place), at batch 2 also those with inputs left to copy
YOLO_VIEWS = {1: (8, 10), 2: (8, 13)}


@pytest.mark.parametrize("batch", sorted(YOLO_VIEWS))
def test_yolo_v10n_views_against_oracle(gpu, monkeypatch, batch):
    """The YOLOv10n-style detector (160x160): the C2f Splits and the Concats
    the views cover skip their copies; all four outputs equal the copying
    path bit for bit, and each image's detections match the oracle's."""
    from spinnv2_amd.runtime import Model
    from tests.helpers import check_detections

    g = models.yolo_v10n(batch=batch, image=160, topk=50)
    blob = write_spk(g, "mi355x")
    xs = rng_inputs(g, dist="uniform")
    runs = {}
    for flag in ("1", "0"):
        monkeypatch.setenv("SPKV2_CONCAT_VIEWS", flag)
        with Model(blob) as m:
            m.set_input(0, xs[0])
            m.run()
            runs[flag] = ([m.get_output(i) for i in range(4)], [m.kernel_name(i) for i in range(len(g.nodes))])
    got, names = runs["1"]
    assert (names.count("split_views"), names.count("concat_views")) == YOLO_VIEWS[batch], names
    # the detection head: three level Concats and the level join elided, the
    # three Reshapes too; the convs wrote the [N, 144, L] buffer in place
    assert (names.count("concat_elided"), names.count("copy_elided")) == (4, 3), names
    assert "concat_elided" not in runs["0"][1]
    for a_, b_ in zip(got, runs["0"][0]):
        np.testing.assert_array_equal(a_.view(np.uint32), b_.view(np.uint32))
    from oracle.spk_exec import OracleExecutor

    want = [np.asarray(o) for o in OracleExecutor(blob).run(*xs)]
    for n in range(batch):  # anchor indices repeat across images: one image at a time
        check_detections([a.reshape(w.shape)[n] for a, w in zip(got, want)], [w[n] for w in want])


@pytest.mark.parametrize("force", [("SPKV2_CONV_SPLITK", "3"), ("SPKV2_CONV_CFG", "18"), ("SPKV2_CONV_CFG", "12"),
                                   ("SPKV2_CONV_CFG", "24")],
                         ids=["splitk3", "thin32", "skinny", "window16"])
def test_yolo_head_views_every_epilogue(gpu, monkeypatch, force):
    """The detection head's convs write the [N, 144, L] buffer with channel
    stride L through every epilogue that can take them (split-K partials
    summed by splitk_epilogue, the thin and the skinny kernels and the
    skinny kernel's row-window form): outputs equal the copying path bit for
    bit."""
    from spinnv2_amd.runtime import Model

    monkeypatch.setenv(*force)
    g = models.yolo_v10n(batch=2, image=160, topk=50)
    blob = write_spk(g, "mi355x")
    xs = rng_inputs(g, dist="uniform")
    print(f"[views] yolo head {force}", flush=True)
    runs = {}
    for flag in ("1", "0"):
        monkeypatch.setenv("SPKV2_CONCAT_VIEWS", flag)
        with Model(blob) as m:
            m.set_input(0, xs[0])
            m.run()
            runs[flag] = ([m.get_output(i) for i in range(4)], [m.kernel_name(i) for i in range(len(g.nodes))])
    assert runs["1"][1].count("concat_elided") == 4, runs["1"][1]
    for a_, b_ in zip(runs["1"][0], runs["0"][0]):
        np.testing.assert_array_equal(a_.view(np.uint32), b_.view(np.uint32))


def test_split_pad_handoff_bit_identical(gpu, monkeypatch):
    """A padded 3x3 conv reading one output of a channel Split takes its
    zero-padded input from the conv the Split cuts (that conv stores the
    channel range into it): every output equals the copying path bit for
    bit, with and without the channel-slice views."""
    g = _c2f_graph(batch=2, widths=(32, 64))
    blob = write_spk(g, "mi355x")
    xs = rng_inputs(g)
    split_outs = {t for n in g.nodes if n.op_type == "Split" for t in n.outputs}
    readers = [n.id for n in g.nodes if n.op_type == "Conv" and n.inputs[0] in split_outs]
    assert readers
    outs = {}
    for views in ("1", "0"):
        monkeypatch.setenv("SPKV2_CONCAT_VIEWS", views)
        for flag in ("1", "0"):
            monkeypatch.setenv("SPKV2_PAD_HANDOFF", flag)
            out, names = _run(blob, xs, len(g.nodes))
            outs[views, flag] = out
            if flag == "1":
                assert all(names[i].endswith("+handoff") for i in readers), [names[i] for i in readers]
            else:
                assert not any(names[i].endswith("+handoff") for i in readers)
    for k, v in outs.items():
        np.testing.assert_array_equal(v.view(np.uint32), outs["0", "0"].view(np.uint32), err_msg=str(k))


@pytest.mark.parametrize("batch", [1, 2])
def test_unaligned_add_view_scalar_path(gpu, monkeypatch, batch):
    """An Add placed in a Concat buffer at a channel offset whose byte
    offset is not a multiple of 16 (2 channels of 5x5 planes before it) and
    with odd image strides: binary_run takes its scalar image-strided kernel
    (binary_img1), bit-identical to the copying path."""
    p = models.Params(5)
    g = Graph("unaligned_add_view")
    x = g.input("x", [batch, 3, 5, 5])
    a = g.conv(x, p.he((2, 3, 1, 1)), p.normal(2, 0.01))
    # Relu on both convs keeps the Add from fusing into either
    b1 = g.relu(g.conv(x, p.he((4, 3, 3, 3)), p.normal(4, 0.01), pad=1))
    b2 = g.relu(g.conv(x, p.he((4, 3, 1, 1)), p.normal(4, 0.01)))
    s = g.add(b1, b2)
    z = g.concat([a, s], axis=1)
    y = g.conv(z, p.he((3, 6, 3, 3)), p.normal(3, 0.01), pad=1)
    g.mark_output(y)
    run_default_pipeline(g)
    blob = write_spk(g, "mi355x")
    xs = rng_inputs(g)
    print(f"[views] unaligned Add view batch {batch}", flush=True)
    monkeypatch.setenv("SPKV2_CONCAT_VIEWS", "1")
    on, names_on = _run(blob, xs, len(g.nodes))
    monkeypatch.setenv("SPKV2_CONCAT_VIEWS", "0")
    off, names_off = _run(blob, xs, len(g.nodes))
    np.testing.assert_array_equal(on.view(np.uint32), off.view(np.uint32))
    assert "Add" in [n.op_type for n in g.nodes]
    assert "binary_img1" in names_on or batch == 1, names_on
    assert "binary_img1" not in names_off
    want = run_oracle(blob, xs)[0]
    assert tnorm_err(on, want) <= FP32_TOL
