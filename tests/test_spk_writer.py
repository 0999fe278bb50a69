"""The repo's SPK writer, graph passes and arena planner (host logic, no GPU).

The oracle reads packages with its own parser (oracle/spk_exec.py), so a
writer bug shows up as a disagreement here or in the golden tests rather
than being shared by both sides.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle.spk_exec import OracleExecutor, Package
from spinnv2_amd.runtime import load_library
from spinnv2_amd.spk import format as F
from spinnv2_amd.spk import models, write_spk
from spinnv2_amd.spk.graph import Graph
from spinnv2_amd.spk.kernel_spec import select_kernel_specs
from spinnv2_amd.spk.passes import run_default_pipeline
from spinnv2_amd.spk.planner import SHAPE_ONLY, plan_memory


@pytest.fixture(scope="module")
def resnet18():
    return models.resnet(18, 1, image=64, classes=10)


def test_record_sizes_match_the_c_header():
    # runtime/include/spkv2_format.h of the reference; include/spkv2_format.h static_asserts the same
    assert (F.HEADER.size, F.SECTION.size, F.TENSOR.size, F.NODE.size, F.ATTR.size, F.MEMORY_PLAN.size,
            F.KERNEL_SPEC.size, F.QUANT_PARAM.size, F.PROTECTION.size) == (68, 32, 68, 76, 124, 36, 44, 20, 28)


def test_writer_is_deterministic_and_checksummed(resnet18):
    a = write_spk(resnet18, "mi355x")
    b = write_spk(resnet18, "mi355x")
    assert a == b
    hdr = F.HEADER.unpack_from(a, 0)
    assert hdr[0] == 0x32564B50 and hdr[1] == 0 and hdr[2] == 3 and hdr[-1] == 1
    secs = [F.SECTION.unpack_from(a, hdr[4] + i * F.SECTION.size) for i in range(hdr[5])]
    ck = [s for s in secs if s[0] == F.SECTION_CHECKSUM][0]
    stored = int.from_bytes(a[ck[2]:ck[2] + 4], "little")
    assert stored == load_library().spkv2_fnv1a32(a[:ck[2]], ck[2])
    for s in secs:
        assert s[2] % max(s[4], 1) == 0 and s[2] + s[3] <= len(a)


def test_independent_parser_agrees(resnet18):
    blob = write_spk(resnet18, "mi355x")
    pkg = Package(blob)
    assert len(pkg.nodes) == len(resnet18.nodes)
    for t in resnet18.tensors:
        assert list(pkg.tensors[t.id].shape) == list(t.shape)
    for t in resnet18.tensors:
        if t.role == "weight":
            np.testing.assert_array_equal(pkg.weights[t.id].ravel(), t.data.ravel())


def test_default_pipeline_fuses_resnet_blocks():
    g = models.resnet(18, 1, image=64, classes=10)
    ops = [n.op_type for n in g.nodes]
    assert ops.count("Conv") == 20
    assert "BatchNormalization" not in ops and "Relu" not in ops and "Add" not in ops
    convs = [n for n in g.nodes if n.op_type == "Conv"]
    assert sum(1 for n in convs if len(n.inputs) == 4) == 8          # block tails carry the residual
    assert all(n.attrs.get("fused_activation") == "Relu" for n in convs if len(n.inputs) == 4)


def test_batchnorm_fold_matches_unfolded_float64():
    rng = np.random.default_rng(5)
    w = rng.standard_normal((6, 3, 3, 3)).astype(np.float32)
    b = rng.standard_normal(6).astype(np.float32)
    gamma = rng.uniform(0.5, 1.5, 6).astype(np.float32)
    beta = rng.normal(0, 0.1, 6).astype(np.float32)
    mean = rng.normal(0, 0.1, 6).astype(np.float32)
    var = rng.uniform(0.5, 1.5, 6).astype(np.float32)
    g = Graph("bn")
    x = g.input("x", [1, 3, 8, 8])
    y = g.conv(x, w, b, pad=1)
    y = g.batchnorm(y, gamma, beta, mean, var)
    g.mark_output(y)
    run_default_pipeline(g)
    assert [n.op_type for n in g.nodes] == ["Conv"]
    xin = rng.standard_normal((1, 3, 8, 8)).astype(np.float32)
    got = OracleExecutor(write_spk(g, "mi355x")).run(xin)[0]
    # unfolded: conv in float64, then BN
    xp = np.pad(xin.astype(np.float64), ((0, 0), (0, 0), (1, 1), (1, 1)))
    conv = np.zeros((1, 6, 8, 8))
    for kh in range(3):
        for kw in range(3):
            conv[0] += np.einsum("chw,mc->mhw", xp[0, :, kh:kh + 8, kw:kw + 8], w[:, :, kh, kw].astype(np.float64))
    conv += b[:, None, None]
    want = (conv - mean[:, None, None]) / np.sqrt(var[:, None, None] + 1e-5) * gamma[:, None, None] + beta[:, None, None]
    np.testing.assert_allclose(got, want, rtol=0, atol=2e-5 * np.abs(want).max())


def _alias_groups(g):
    parent = {t.id: t.id for t in g.tensors}

    def find(a):
        while parent[a] != a:
            parent[a] = parent[parent[a]]
            a = parent[a]
        return a

    for n in g.nodes:
        if n.op_type in SHAPE_ONLY or n.op_type in ("Relu", "Concat"):
            for i in n.inputs:
                parent[find(i)] = find(n.outputs[0])
    return find


@pytest.mark.parametrize("builder", ["lenet", "resnet18", "resnet50", "concat"])
def test_arena_plan_has_no_live_overlap(builder):
    if builder == "lenet":
        g = models.lenet()
    elif builder == "resnet18":
        g = models.resnet(18, 2, image=64, classes=10)
    elif builder == "resnet50":
        g = models.resnet(50, 1, image=64, classes=10)
    else:
        g = Graph("concat")
        x = g.input("x", [1, 4, 6, 6])
        p = models.Params(1)
        a = g.conv(x, p.he((8, 4, 3, 3)), None, pad=1)
        b = g.conv(x, p.he((4, 4, 1, 1)), None)
        c = g.concat([a, b], axis=1)
        g.mark_output(g.relu(c))
    plan = plan_memory(g)
    find = _alias_groups(g)
    ents = list(plan.entries.values())
    for i, e in enumerate(ents):
        assert e.offset % 16 == 0
        assert e.offset + e.size <= plan.arena_bytes or e.memory_class != "ACTIVATION_ARENA"
        for f in ents[i + 1:]:
            if e.memory_class != f.memory_class or e.memory_class == "WEIGHT":
                continue
            live = e.first_use <= f.last_use and f.first_use <= e.last_use
            bytes_overlap = e.offset < f.offset + f.size and f.offset < e.offset + e.size
            if live and bytes_overlap:
                assert find(e.tensor_id) == find(f.tensor_id), (builder, e, f)
    assert plan.arena_bytes <= plan.naive_bytes


def test_kernel_specs_per_profile(resnet18):
    specs, by_node, _ = select_kernel_specs(resnet18, "mi355x")
    for n in resnet18.nodes:
        s = by_node.get(n.id)
        if n.op_type == "Conv":
            assert s.backend == "mi355x" and s.kind == "implicit_gemm_f32"
        elif n.op_type == "Gemm":
            assert s.backend == "mi355x" and s.kind == "gemm_f32"
    _, by_node, _ = select_kernel_specs(resnet18, "cpu_generic")
    # reference compiler/planner/kernel_spec.py:161-163: group==1 conv -> bnns_fp32 under cpu_generic
    assert all(by_node[n.id].kind == "bnns_fp32" for n in resnet18.nodes if n.op_type == "Conv")
    _, by_node, _ = select_kernel_specs(resnet18, "cpu_ref")
    assert all(s.backend == "ref" for s in by_node.values())


def test_arm_profiles_conv_kinds_and_scratch():
    """cpu_arm_neon picks Winograd F(4,3) for 3x3/s1/p1 convs of at least
    8x8 outputs and 4 tiles (reference kernel_spec.py:188-206), with scratch
    36*(C+M)*tiles*4 (kernel_spec.py:255-263); the experimental profile
    picks F(2,3) (scratch 16*(C+M)*tiles*4 with 2x2 tiles, :244-254) and the
    3x3/s2 direct conv (no scratch) for convs without a fused residual."""
    g = models.resnet(18, 1, image=64, classes=10)
    _, arm, _ = select_kernel_specs(g, "cpu_arm_neon")
    _, exp, _ = select_kernel_specs(g, "cpu_arm_neon_exp")
    seen = set()
    for n in g.nodes:
        if n.op_type != "Conv":
            continue
        x, w, y = (g.tensors[t].shape for t in (n.inputs[0], n.inputs[1], n.outputs[0]))
        s1p1 = w[2] == 3 and n.attrs["strides"] == [1, 1] and n.attrs["pads"] == [1, 1, 1, 1]
        s2p1 = w[2] == 3 and n.attrs["strides"] == [2, 2] and n.attrs["pads"] == [1, 1, 1, 1]
        t4 = ((y[2] + 3) // 4) * ((y[3] + 3) // 4)
        if s1p1 and y[2] >= 8 and t4 >= 4:
            assert arm[n.id].kind == "winograd_f43"
            assert arm[n.id].scratch_bytes == 36 * (x[1] + w[0]) * t4 * 4
        else:
            assert arm[n.id].kind in ("im2col_gemm", "pointwise_1x1"), arm[n.id].kind
        plain = len(n.inputs) < 4
        t2 = ((y[2] + 1) // 2) * ((y[3] + 1) // 2)
        if s1p1 and plain:
            assert exp[n.id].kind == "winograd_3x3s1"
            assert exp[n.id].scratch_bytes == 16 * (x[1] + w[0]) * t2 * 4
        elif s2p1 and plain:
            assert exp[n.id].kind == "conv3x3s2_direct" and exp[n.id].scratch_bytes == 0
        seen |= {arm[n.id].kind, exp[n.id].kind}
        assert arm[n.id].backend == exp[n.id].backend == "simd"
    assert {"winograd_f43", "winograd_3x3s1", "conv3x3s2_direct", "im2col_gemm"} <= seen


def test_spk_round_trips_through_the_runtime_loader(resnet18):
    import ctypes

    lib = load_library()
    blob = write_spk(resnet18, "mi355x")
    buf = ctypes.create_string_buffer(blob, len(blob))
    ctx = ctypes.c_void_p()
    assert lib.spkv2_load_memory(buf, len(blob), ctypes.byref(ctx)) == 0
    size = ctypes.c_size_t()
    assert lib.spkv2_get_output_size(ctx, 0, ctypes.byref(size)) == 0
    assert size.value == 10 * 4
    rec = lib.spkv2_ctx_tensor_record(ctx, 0)
    assert rec
    lib.spkv2_free(ctx)
