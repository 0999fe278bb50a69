"""Protected execution on the MI355X runtime against the reference runtime.

tests/golden/reliability/ holds what the reference runtime did on each case
(tests/golden/reliability/make_reliability.py): fault-event and run return
codes, cumulative reliability stats, range observations and outputs.  The
mi355x package of the same graph and protection plan replays the same
sequence on the GPU (bit flips by a device kernel, range checks and DMR
compares on device, reference runtime/core/executor.c:377-498).  Codes,
stats and observation counts must be equal; outputs and observed extrema
bit-exact for the Relu cases and within the fp32 tolerance for the
networks.
"""

from __future__ import annotations

import numpy as np
import pytest

from .helpers import FP32_TOL, tnorm_err
from .reliability_cases import gpu_adapter, load, package, replay

CASES, ARRAYS = load()


def close(got_bits: int, want_bits: int, exact: bool) -> bool:
    if got_bits == want_bits:
        return True
    if exact:
        return False
    a, b = (float(np.uint32(v).view(np.float32)) for v in (got_bits, want_bits))
    return bool(np.isfinite(a) and np.isfinite(b) and abs(a - b) <= FP32_TOL * max(abs(b), 1.0))


@pytest.mark.gpu
@pytest.mark.parametrize("case", CASES, ids=[c["name"] for c in CASES])
def test_protected_execution_matches_reference(gpu, case):
    from spinnv2_amd.runtime import Model

    print(f"[reliability] {case['name']}", flush=True)
    g, blob = package(case, "mi355x")
    with Model(blob) as m:
        runs, outs = replay(case, g, gpu_adapter(m))
    for n, (got, want) in enumerate(zip(runs, case["runs"])):
        where = f"run {n}"
        assert (got["fault_rc"], got["rc"], got["outputs"]) == (want["fault_rc"], want["rc"], want["outputs"]), where
        assert got["stats"] == want["stats"], where
        for node, (lo, hi, count) in want["ranges"].items():
            glo, ghi, gcount = got["ranges"][node]
            assert gcount == count, (where, node)
            assert close(glo, lo, case["exact"]) and close(ghi, hi, case["exact"]), (where, node, glo, lo, ghi, hi)
    assert sorted(outs) == sorted(k for k in ARRAYS if k.startswith(case["name"] + "__"))
    for key, got in outs.items():
        want = ARRAYS[key]
        if case["exact"]:
            np.testing.assert_array_equal(got, want, err_msg=key)
        else:
            assert tnorm_err(got.view(np.float32), want.view(np.float32)) <= FP32_TOL, key
