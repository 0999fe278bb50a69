"""MI355X runtime against the reference runtime's own outputs.

The fixtures in tests/golden/ hold what the reference SPINNV2 C runtime
computed on the same graphs and inputs (tests/golden/make_golden.py); here
the `mi355x` package of each graph runs on the GPU through the C ABI.
Bar: bit-exact for selection / copy / single-add ops, fp32 tensor-normalized
error <= 1e-4 for contractions, plus top-1 agreement for the networks.
"""

from __future__ import annotations

import numpy as np
import pytest

from spinnv2_amd.spk import write_spk

from .golden_cases import load_cases
from .helpers import FP32_TOL, check_detections, run_gpu, tnorm_err

CASES = load_cases()
NETWORKS = {"lenet", "resnet18_32px", "resnet50_32px"}
DETECTORS = {"yolov10n_160"}


@pytest.mark.gpu
@pytest.mark.parametrize("case", CASES, ids=[c.name for c in CASES])
def test_mi355x_matches_reference_runtime(gpu, case):
    """The mi355x package of every fixture; for the ARM-profile fixtures also
    the very package the reference ran (conv kinds 7/8/9 and SIMD im2col
    dispatched to the device kernels unchanged)."""
    print(f"[golden] {case.name}", flush=True)
    blobs = [write_spk(case.graph(), "mi355x")]
    if case.optimized:
        blobs.append(write_spk(case.graph(), case.profile))
    for blob in blobs:
        _check(case, run_gpu(blob, case.inputs, outputs=len(case.all_expected)))


def _check(case, outs):
    if case.name in DETECTORS:
        check_detections(outs, case.all_expected)
        return
    for got, want in zip(outs, case.all_expected):
        got = got.ravel()
        assert got.shape == want.shape
        if case.exact:
            np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))
        else:
            assert tnorm_err(got, want) <= FP32_TOL
    got = outs[0].ravel()
    if case.name in NETWORKS or case.builder == "resnet":
        rows = got.reshape(case.inputs[0].shape[0], -1)
        want = case.expected.reshape(rows.shape)
        assert (rows.argmax(axis=1) == want.argmax(axis=1)).all()
