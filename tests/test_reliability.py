"""Protection plans in packages, and the fixtures of protected execution.

The encoding follows the reference compiler (compiler/reliability/
protection_plan.py:65-81, compiler/packager/spk_writer.py:140-200): 28-byte
records after the quantization section, infinite bounds stored as
+-FLT_MAX, the DMR copies placed after the kernels' scratch arena and the
header's scratch size grown by two copies of the largest DMR output.  The
fixtures are replayed on the reference runtime itself when it was built
here (oracle/_ref), which pins both this writer's encoding and the
fixtures; the MI355X runtime replays the same fixtures on the GPU.
"""

from __future__ import annotations

import math

import numpy as np
import pytest

from spinnv2_amd.spk import Protection, models, write_spk
from spinnv2_amd.spk import format as F

from .reliability_cases import load, package, ref_adapter, replay

FLT_MAX = 3.4028234663852886e38


def sections(blob: bytes) -> list[tuple]:
    hdr = F.HEADER.unpack_from(blob, 0)
    return [F.SECTION.unpack_from(blob, hdr[4] + i * F.SECTION.size) for i in range(hdr[5])]


def protection_records(blob: bytes) -> list[tuple]:
    sec = [s for s in sections(blob) if s[0] == F.SECTION_PROTECTION_PLAN]
    if not sec:
        return []
    (s,) = sec
    assert s[3] % F.PROTECTION.size == 0
    return [F.PROTECTION.unpack_from(blob, s[2] + i * F.PROTECTION.size) for i in range(s[3] // F.PROTECTION.size)]


def test_protection_section_encoding():
    g = models.lenet()
    plain = write_spk(g, "mi355x")
    blob = write_spk(g, "mi355x", protection=[
        Protection(0, "range_guard_rerun", 0.0, 6.5),
        Protection(2, "dmr_compare_rerun"),
        Protection(5, "range_guard_rerun", -math.inf, 100.0),
        Protection(9, "dmr_compare_rerun")])
    recs = protection_records(blob)
    assert protection_records(plain) == []
    kernel_scratch = F.HEADER.unpack_from(plain, 0)[13]
    out = {n: g.nodes[n].outputs[0] for n in (0, 2, 5, 9)}
    assert [(r[0], r[1], r[2], r[3]) for r in recs] == [(0, out[0], 1, 0), (2, out[2], 2, 0), (5, out[5], 1, 0),
                                                       (9, out[9], 2, 0)]
    assert (recs[0][4], recs[0][5]) == (0.0, 6.5)
    assert np.float32(recs[1][4]) == np.float32(-FLT_MAX) and np.float32(recs[1][5]) == np.float32(FLT_MAX)
    assert np.float32(recs[2][4]) == np.float32(-FLT_MAX) and recs[2][5] == 100.0
    # DMR copies start after the kernels' scratch; range guards use none
    assert [r[6] for r in recs] == [0, kernel_scratch, 0, kernel_scratch]
    dmr_bytes = max(2 * g.tensors[out[n]].size_bytes for n in (2, 9))
    assert F.HEADER.unpack_from(blob, 0)[13] == kernel_scratch + dmr_bytes
    # after the quantization section (if any), before the string table, 8-byte aligned
    order = [s[0] for s in sections(blob)]
    assert order.index(F.SECTION_PROTECTION_PLAN) == order.index(F.SECTION_STRING_TABLE) - 1
    sec = [s for s in sections(blob) if s[0] == F.SECTION_PROTECTION_PLAN][0]
    assert sec[2] % 8 == 0 and sec[4] == 8


def test_protection_rejects_what_the_runtime_cannot_guard():
    g = models.index_op("Split", [1, 6, 4, 4], axis=1, sizes=[2, 4])
    with pytest.raises(ValueError):
        write_spk(g, "mi355x", protection=[Protection(0, "range_guard_rerun")])    # two outputs
    g = models.lenet()
    with pytest.raises(ValueError):
        write_spk(g, "mi355x", protection=[Protection(0, "range_guard_rerun", 2.0, 1.0)])
    with pytest.raises(ValueError):
        write_spk(g, "mi355x", protection=[Protection(0, "dmr_compare_rerun"), Protection(0, "range_guard_rerun")])


def test_fixtures_cover_the_reference_scenario():
    """runtime/tests/test_reliability.c: Relu on [-1, 2, 3, 4], sign flip of
    element 1 after the first invocation -> one fault injected, detected,
    recovered by one rerun, output [0, 2, 3, 4]."""
    cases, arrays = load()
    case = next(c for c in cases if c["name"] == "relu_range_guard_sign_flip")
    (run,) = case["runs"]
    assert run["fault"] == dict(node_id=0, tensor_id=1, element_index=1, bit_index=31, invocation_index=1,
                                seed=2026, enabled=1)
    assert run["rc"] == 0 and run["stats"] == dict(injected_faults=1, detected_faults=1, recovered_faults=1,
                                                   unrecovered_faults=0, rerun_count=1)
    np.testing.assert_array_equal(arrays["relu_range_guard_sign_flip__0__0"].view(np.float32), [0, 2, 3, 4])


REF_CASES = load()[0]


@pytest.mark.parametrize("case", REF_CASES, ids=[c["name"] for c in REF_CASES])
def test_reference_runtime_reproduces_fixture(case):
    from oracle.ref_runtime import RefModel, available

    if not available():
        pytest.skip("reference runtime not built here (make -C oracle ref)")
    _, arrays = load()
    g, blob = package(case, "cpu_ref")
    m = RefModel(blob)
    try:
        runs, out = replay(case, g, ref_adapter(m))
    finally:
        m.close()
    assert runs == case["runs"]
    for k, v in out.items():
        np.testing.assert_array_equal(v, arrays[k])
