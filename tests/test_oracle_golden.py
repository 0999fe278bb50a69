"""The CPU oracle against the reference runtime's own outputs (no GPU).

Every fixture in tests/golden/ holds the output of the reference SPINNV2 C
runtime (runtime/core + runtime/kernels/reference, built from its sources by
oracle/Makefile) on a package of the same graph.  The oracle restates those
kernels including the rounding of the reference's release build, so it
must agree bit for bit.  When oracle/_ref is built (this container), the
same check also runs live on freshly seeded inputs.
"""

from __future__ import annotations

import numpy as np
import pytest

from tests.golden_cases import load_cases
from oracle.spk_exec import OracleExecutor
from spinnv2_amd.spk import models, write_spk

CASES = load_cases()


def test_fixture_set_is_complete():
    names = {c.name for c in CASES}
    assert len(CASES) >= 56
    for required in ("lenet", "resnet18_32px", "resnet50_32px", "conv2", "gemm2", "op0_MaxPool", "op6_Resize",
                     "op7_Softmax", "op2_Add"):
        assert required in names


@pytest.mark.parametrize("case", CASES, ids=[c.name for c in CASES])
def test_oracle_matches_reference_bitwise(case):
    """Bit for bit against the reference kernels the oracle restates; within
    the fp32 tolerance (same top-1 for networks) where the reference ran its
    optimized Winograd / AVX2 kernels on an ARM-profile package."""
    from tests.helpers import FP32_TOL, tnorm_err

    blob = write_spk(case.graph(), "mi355x")
    outs = OracleExecutor(blob).run(*case.inputs)
    assert len(outs) == len(case.all_expected)
    for got, want in zip(outs, case.all_expected):
        got = got.ravel()
        assert got.shape == want.shape
        if case.optimized:
            assert tnorm_err(got, want) <= FP32_TOL
            assert np.argmax(got) == np.argmax(want)
        else:
            np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))


def test_arm_profile_packages_carry_every_conv_kind():
    """The ARM-profile fixtures are packages with conv kinds 7, 8 and 9 (and
    im2col on SIMD), the codes of reference spkv2_format.h:130-132."""
    from spinnv2_amd.spk import format as F
    from spinnv2_amd.spk.kernel_spec import select_kernel_specs

    kinds = set()
    for c in CASES:
        if c.optimized:
            _, by_node, _ = select_kernel_specs(c.graph(), c.profile)
            kinds |= {F.KIND[s.kind] for s in by_node.values() if s.backend == "simd"}
    assert {7, 8, 9, 3} <= kinds, kinds


def _ref_available() -> bool:
    from oracle.ref_runtime import available

    return available()


@pytest.mark.skipif(not _ref_available(), reason="oracle/_ref/libspkv2_ref.so not built (needs /root/reference)")
@pytest.mark.parametrize("seed", [7, 1234])
@pytest.mark.parametrize("conv", [
    dict(n=2, cin=12, h=11, w=13, cout=20, k=3, stride=2, pad=1, act="Relu", residual=False),
    dict(n=1, cin=9, h=8, w=8, cout=5, k=5, stride=1, pad=2, dilation=1, act="Silu"),
    dict(n=2, cin=6, h=9, w=9, cout=6, k=3, stride=1, pad=1, act="Relu", residual=True),
])
def test_oracle_matches_live_reference_conv(conv, seed):
    from oracle.ref_runtime import RefModel

    g = models.single_conv(**conv, seed=seed)
    xs = [models.make_input(g.tensors[t].shape, seed + i) for i, t in enumerate(g.inputs)]
    ref = RefModel(write_spk(g, "cpu_ref"))
    want = ref.run(*xs)
    ref.close()
    got = OracleExecutor(write_spk(g, "mi355x")).run(*xs)[0].ravel()
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.skipif(not _ref_available(), reason="oracle/_ref/libspkv2_ref.so not built (needs /root/reference)")
def test_oracle_matches_live_reference_simd_conv_within_tolerance():
    """The reference's own AVX2 im2col+SGEMM conv (cpu_generic without the
    BNNS token) differs from its naive conv by reassociation only; the
    oracle is within the fp32 tolerance of it too."""
    from oracle.ref_runtime import RefModel

    from tests.helpers import FP32_TOL, tnorm_err

    g = models.single_conv(2, 32, 14, 14, 48, 3, 1, 1)
    xs = [models.make_input(g.tensors[t].shape, 99 + i) for i, t in enumerate(g.inputs)]
    ref = RefModel(write_spk(g, "cpu_generic_nobnns"))
    want = ref.run(*xs)
    ref.close()
    got = OracleExecutor(write_spk(g, "mi355x")).run(*xs)[0].ravel()
    assert tnorm_err(got, want) <= FP32_TOL
