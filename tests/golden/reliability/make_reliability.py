"""Writes tests/golden/reliability/ from the reference SPINNV2 C runtime.

Each case is a package with a protection plan (range_guard_rerun /
dmr_compare_rerun records, compiler/reliability/protection_plan.py:65-81)
and a sequence of runs, each optionally armed with a bit-flip fault event
(runtime/core/executor.c:377-398).  Per run the fixture keeps what the
reference runtime (oracle/_ref/libspkv2_ref.so, built from
/root/reference/runtime by `make -C oracle ref`) returned: the
spkv2_set_fault_event and spkv2_run codes, the cumulative reliability stats
and the range observations of the protected nodes (fp32 bit patterns) in
cases.json, the graph outputs in outputs.npz (key
"<case>__<run>__<output>").  The first case is the reference's own
runtime/tests/test_reliability.c scenario.

    python tests/golden/reliability/make_reliability.py   # rewrites cases.json, outputs.npz

Needs /root/reference; the GPU box never runs this.
"""

from __future__ import annotations

import json
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent.parent.parent
sys.path.insert(0, str(ROOT))

from oracle.ref_runtime import RefModel, available  # noqa: E402
from spinnv2_amd.spk import write_spk  # noqa: E402
from tests.reliability_cases import build, case_input, package, ref_adapter, replay  # noqa: E402

OUT = HERE / "cases.json"
OUT_ARRAYS = HERE / "outputs.npz"


def fault(node, tensor, element, bit, invocation=1, seed=2026, enabled=1) -> dict:
    return dict(node_id=node, tensor_id=tensor, element_index=element, bit_index=bit,
                invocation_index=invocation, seed=seed, enabled=enabled)


def replay_ref(case: dict, arrays: dict) -> dict:
    g, blob = package(case, "cpu_ref")
    m = RefModel(blob)
    runs, out = replay(case, g, ref_adapter(m))
    m.close()
    arrays.update(out)
    return {**case, "runs": runs}


def relu_cases() -> list[dict]:
    base = dict(builder="single_op", kwargs=dict(op="Relu", shape=[4]), exact=True)
    x = {"values": [-1.0, 2.0, 3.0, 4.0]}
    rg = [dict(node_id=0, mode="range_guard_rerun", lower=0.0, upper=10.0)]
    dmr = [dict(node_id=0, mode="dmr_compare_rerun", lower=float("-inf"), upper=float("inf"))]
    return [
        # runtime/tests/test_reliability.c: sign flip of element 1, caught by
        # the range guard, recovered by the rerun
        dict(base, name="relu_range_guard_sign_flip", protection=rg,
             runs=[dict(fault=fault(0, 1, 1, 31), input=x)]),
        dict(base, name="relu_dmr_first_copy", protection=dmr,
             runs=[dict(fault=fault(0, 1, 1, 31), input=x)]),
        dict(base, name="relu_dmr_second_copy", protection=dmr,
             runs=[dict(fault=fault(0, 1, 2, 5, invocation=2), input=x)]),
        dict(base, name="relu_dmr_no_third_invocation", protection=dmr,
             runs=[dict(fault=fault(0, 1, 0, 30, invocation=3), input=x)]),
        dict(base, name="relu_range_guard_undetected", protection=rg,
             runs=[dict(fault=fault(0, 1, 3, 0), input=x)]),
        dict(base, name="relu_range_guard_tight_bounds",
             protection=[dict(node_id=0, mode="range_guard_rerun", lower=0.0, upper=3.0)],
             runs=[dict(fault=None, input=x), dict(fault=fault(0, 1, 2, 31, invocation=2), input=x)]),
        dict(base, name="relu_unprotected", protection=[],
             runs=[dict(fault=fault(0, 1, 2, 30), input=x), dict(fault=None, input=x)]),
        dict(base, name="relu_fault_errors", protection=rg,
             runs=[dict(fault=fault(0, 1, 1, 32), input=x),                 # bit index out of range
                   dict(fault=fault(1, 1, 1, 3), input=x),                  # no such node
                   dict(fault=fault(0, 2, 1, 3), input=x),                  # no such tensor
                   dict(fault=fault(0, 0, 1, 3), input=x),                  # not the node's output
                   dict(fault=fault(0, 1, 4, 3), input=x),                  # element out of range
                   dict(fault=fault(0, 1, 1, 31, invocation=0), input=x),   # never fires
                   dict(fault=fault(0, 1, 1, 31, enabled=0), input=x),      # disarmed
                   dict(fault=None, input=x)]),
        dict(base, name="relu_range_observations", protection=rg,
             runs=[dict(fault=None, input=x),
                   dict(fault=None, input={"values": [-5.0, 0.5, 7.0, 1.0]}),
                   dict(fault=None, input={"values": [-0.0, 9.5, 0.25, 0.0]}),
                   dict(fault=None, input=x, reset_ranges=True, reset_stats=True)]),
    ]


def lenet_case() -> dict:
    """LeNet with the first conv range-guarded (its output also a graph
    output, so the faulted tensor is compared too), the second conv under
    DMR, the first Gemm range-guarded without a fault, and faults placed
    from the reference's own values."""
    case = dict(name="lenet_protected", builder="lenet", kwargs={}, exact=False, extra_outputs=[3, 7])
    g, _ = build(dict(case, protection=[]))
    m = RefModel(write_spk(g, "cpu_ref"))
    x = case_input(g, {"seed": 7})
    m.run(*x)
    conv1 = m.output(1)
    gemm_in = m.output(2)
    m.close()
    # a relu output in (0.25, 1): flipping bit 30 multiplies it by 2^128
    e1 = int(np.argmin(np.abs(conv1 - 0.6)))
    assert 0.25 < conv1[e1] < 1.0
    e2 = int(np.argmax(gemm_in))

    prot = [dict(node_id=0, mode="range_guard_rerun", lower=-1.0, upper=float(conv1.max()) * 1.5 + 1.0),
            dict(node_id=2, mode="dmr_compare_rerun", lower=float("-inf"), upper=float("inf")),
            dict(node_id=5, mode="range_guard_rerun", lower=-1.0e4, upper=1.0e4)]
    case["protection"] = prot
    case["runs"] = [
        dict(fault=None, input={"seed": 7}),
        dict(fault=fault(0, 3, e1, 30), input={"seed": 7}),
        dict(fault=fault(2, 7, e2, 2), input={"seed": 7}),
        dict(fault=fault(2, 7, e2, 30, invocation=2), input={"seed": 8}),
        dict(fault=fault(7, 16, 5, 23), input={"seed": 7}),       # unprotected Gemm: error propagates
        dict(fault=fault(0, 3, e1, 1), input={"seed": 7}),        # in range: undetected
    ]
    return case


def resnet_case() -> dict:
    """ResNet-18 at 32x32: a protected 3x3 conv (node 2) that would
    otherwise store straight into the next conv's padded input, DMR on a
    conv with a fused residual (node 4).  Faults are placed from the
    reference's values of node 2's output, read from a copy of the graph that
    also returns that tensor."""
    case = dict(name="resnet18_32px_protected", builder="resnet",
                kwargs=dict(depth=18, batch=2, image=32, classes=10), exact=False)
    g, _ = build(dict(case, protection=[]))
    t2 = g.nodes[2].outputs[0]
    t4 = g.nodes[4].outputs[0]
    g.mark_output(t2)
    m = RefModel(write_spk(g, "cpu_ref"))
    m.run(*case_input(g, {"seed": 3}))
    y2 = m.output(1)
    m.close()
    e2 = int(np.argmax(y2 > 0.5))
    assert y2[e2] > 0.5
    case["protection"] = [dict(node_id=2, mode="range_guard_rerun", lower=0.0, upper=1.0e3),
                          dict(node_id=4, mode="dmr_compare_rerun", lower=float("-inf"), upper=float("inf"))]
    case["runs"] = [
        dict(fault=None, input={"seed": 3}),
        dict(fault=fault(2, t2, e2, 31), input={"seed": 3}),        # sign flip of a positive relu output
        dict(fault=fault(4, t4, 17, 12), input={"seed": 3}),
        dict(fault=fault(4, t4, 40, 27, invocation=2), input={"seed": 4}),
    ]
    return case


def main() -> None:
    if not available():
        sys.exit("oracle/_ref/libspkv2_ref.so not built: make -C oracle ref")
    arrays: dict = {}
    cases = [replay_ref(c, arrays) for c in relu_cases() + [lenet_case(), resnet_case()]]
    OUT.write_text(json.dumps({"cases": cases}, indent=1) + "\n")
    np.savez_compressed(OUT_ARRAYS, **arrays)
    print(f"wrote {OUT} and {OUT_ARRAYS} ({len(cases)} cases)")


if __name__ == "__main__":
    main()
