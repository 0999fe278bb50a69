"""The compiler side of the mi355x target: profiles/mi355x.json (the
reference's profile schema, compiler/target/profiles/cpu_generic.json),
kernel selection from its tokens (reference compiler/planner/kernel_spec.py:
71-144), and the device workspace each mi355x kind reserves in its
KernelSpec scratch_bytes, which the runtime then runs out of the package's
scratch arena (caller-provided under spkv2_prepare_with_scratch).
"""

from __future__ import annotations

import json
import os

import numpy as np
import pytest

from spinnv2_amd.spk import format as F
from spinnv2_amd.spk import models, write_spk
from spinnv2_amd.spk import kernel_spec as KS
from spinnv2_amd.spk.kernel_spec import MI355X_PROFILE, select_kernel_specs

from .helpers import rng_inputs


def a256(v: int) -> int:
    return (v + 255) // 256 * 256


def test_profile_lists_every_runtime_op_with_mi355x_kinds():
    assert MI355X_PROFILE["backends"] == ["mi355x"]
    assert set(MI355X_PROFILE["ops"]) == set(F.OP)
    for op, toks in MI355X_PROFILE["ops"].items():
        for t in toks:
            assert t.startswith("mi355x_") and t[len("mi355x_"):] in F.KIND, (op, t)
    assert MI355X_PROFILE["ops"]["Conv"][0] == "mi355x_implicit_gemm_i8"


def test_package_embeds_the_profile():
    blob = write_spk(models.lenet(), "mi355x")
    hdr = F.HEADER.unpack_from(blob, 0)
    secs = {s[0]: s for s in (F.SECTION.unpack_from(blob, hdr[4] + i * F.SECTION.size) for i in range(hdr[5]))}
    s = secs[F.SECTION_TARGET_PROFILE]
    raw = blob[s[2]:s[2] + s[3]]
    assert json.loads(raw) == MI355X_PROFILE
    assert hdr[14] == F.fnv1a32(raw)


def test_selection_follows_the_token_order(monkeypatch):
    g = models.lenet()
    specs, by_node, _ = select_kernel_specs(g, "mi355x")
    conv = by_node[0]
    assert (conv.backend, conv.kind, conv.dtype) == ("mi355x", "implicit_gemm_f32", "fp32")
    assert specs[conv.fallback].kind == "reference"          # the next applicable token
    assert by_node[5].kind == "gemm_f32" and by_node[5].fallback == 0xFFFFFFFF
    assert by_node[1].kind == "device_elementwise"
    prof = json.loads(json.dumps(MI355X_PROFILE))
    prof["ops"]["Conv"] = ["mi355x_reference"]
    monkeypatch.setitem(KS.PROFILES, "mi355x", prof)
    _, by_node, _ = select_kernel_specs(g, "mi355x")
    assert by_node[0].kind == "reference" and by_node[0].scratch_bytes == 0
    del prof["ops"]["MaxPool"]
    with pytest.raises(ValueError, match="does not support op: MaxPool"):
        select_kernel_specs(g, "mi355x")


def test_device_workspace_estimates():
    cap = KS.MI355X_SPLITK_CAP
    # padded 3x3: the zero-padded NCHW copy plus split-K room
    g = models.single_conv(2, 16, 12, 12, 32, 3, stride=1, pad=1)
    _, by_node, scratch = select_kernel_specs(g, "mi355x")
    pad = a256(2 * 16 * 14 * 14 * 4)
    part = min(32 * 32 * 2 * 12 * 12 * 4, cap)
    assert by_node[0].scratch_bytes == pad + part and scratch == pad + part
    # unpadded 1x1: partials only
    g = models.single_conv(1, 64, 7, 7, 128, 1)
    _, by_node, _ = select_kernel_specs(g, "mi355x")
    assert by_node[0].scratch_bytes == min(32 * 128 * 49 * 4, cap)
    # grouped: the direct device conv needs none
    g = models.single_conv(1, 16, 10, 10, 16, 3, pad=1, group=16)
    _, by_node, _ = select_kernel_specs(g, "mi355x")
    assert by_node[0].scratch_bytes == 0
    # large layers hit the per-node cap on the split-K part
    g = models.resnet(101, 64)
    _, by_node, scratch = select_kernel_specs(g, "mi355x")
    stem = by_node[0]
    assert stem.scratch_bytes == a256(64 * 3 * 229 * 229 * 4) + cap    # rows -3..225 of 224 touched
    assert scratch == max(s.scratch_bytes for s in by_node.values())


def test_header_scratch_is_the_largest_spec():
    g = models.resnet(18, 1, image=64, classes=10)
    blob = write_spk(g, "mi355x")
    specs, _, scratch = select_kernel_specs(g, "mi355x")
    assert F.HEADER.unpack_from(blob, 0)[13] == scratch == max(s.scratch_bytes for s in specs)


@pytest.mark.gpu
@pytest.mark.parametrize("forced_split", [None, "64"])
def test_gpu_runs_out_of_caller_scratch(gpu, monkeypatch, forced_split):
    """A caller-provided scratch arena full of NaN bytes: conv, split-K and
    Gemm workspaces live there (nothing may rely on zeroed scratch).  A
    forced split-K of 64 outgrows the compiler's estimate and takes the
    runtime's own workspace instead.  Both runs equal the default run bit
    for bit."""
    from spinnv2_amd.runtime import DeviceBuffer, Model

    print(f"[scratch] forced split {forced_split}", flush=True)
    g = models.resnet(18, batch=2, image=32, classes=10)
    blob = write_spk(g, "mi355x")
    xs = rng_inputs(g, seed=11)
    if forced_split:
        monkeypatch.setenv("SPKV2_CONV_SPLITK", forced_split)
    with Model(blob) as m:
        m.set_input(0, xs[0])
        m.run()
        want = m.get_output(0)
    need = F.HEADER.unpack_from(blob, 0)[13]
    assert need > 0
    scratch = DeviceBuffer(need)
    try:
        scratch.upload(np.full(need, 0xFF, np.uint8))
        m = Model(blob, prepare=False)
        try:
            small = DeviceBuffer(need - 256)
            assert m.prepare_with_scratch(None, small) == -2       # smaller than the header asks
            small.free()
            assert m.prepare_with_scratch(None, scratch) == 0
            m.set_input(0, xs[0])
            m.run()
            got = m.get_output(0)
        finally:
            m.close()
    finally:
        scratch.free()
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))
