"""Protected-execution fixtures (tests/golden/reliability/).

A case is a package (builder call, extra graph outputs, protection plan)
and a sequence of runs, each optionally armed with a bit-flip fault event.
`replay` drives any runtime through the same sequence and returns what it
saw in the fixture's own layout, so the reference runtime (when it was
built here) and the MI355X runtime are checked by the same code.
"""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np

GOLDEN = Path(__file__).resolve().parent / "golden" / "reliability"


def load() -> tuple[list[dict], dict]:
    cases = json.loads((GOLDEN / "cases.json").read_text())["cases"]
    with np.load(GOLDEN / "outputs.npz", allow_pickle=False) as z:
        arrays = {k: z[k] for k in z.files}
    return cases, arrays


def build(case: dict):
    from spinnv2_amd.spk import Protection, models

    kw = dict(case["kwargs"])
    if case["builder"] == "single_op":
        g = models.single_op(kw.pop("op"), kw.pop("shape"), **kw)
    else:
        g = getattr(models, case["builder"])(**kw)
    for t in case.get("extra_outputs", []):
        g.mark_output(t)
    prot = [Protection(p["node_id"], p["mode"], p["lower"], p["upper"]) for p in case["protection"]]
    return g, prot


def package(case: dict, profile: str) -> tuple[object, bytes]:
    from spinnv2_amd.spk import write_spk

    g, prot = build(case)
    return g, write_spk(g, profile, protection=prot or None)


def case_input(g, spec: dict) -> list[np.ndarray]:
    from spinnv2_amd.spk import models

    if "values" in spec:
        return [np.asarray(spec["values"], dtype=np.float32).reshape(g.tensors[g.inputs[0]].shape)]
    return [models.make_input(g.tensors[t].shape, spec["seed"] + i) for i, t in enumerate(g.inputs)]


def f32_bits(v: float) -> int:
    return int(np.float32(v).view(np.uint32))


class Adapter:
    """The calls `replay` makes, bound to one runtime's model object."""

    def __init__(self, set_fault, set_input, run_rc, output, stats, observation, reset_ranges, reset_stats):
        self.set_fault, self.set_input, self.run_rc, self.output = set_fault, set_input, run_rc, output
        self.stats, self.observation = stats, observation
        self.reset_ranges, self.reset_stats = reset_ranges, reset_stats


def replay(case: dict, g, rt: Adapter) -> tuple[list[dict], dict]:
    """Runs the case's sequence; returns per-run records (codes, stats,
    range observations as fp32 bit patterns) and the outputs by fixture
    key."""
    runs, arrays = [], {}
    for r in case["runs"]:
        if r.get("reset_ranges"):
            rt.reset_ranges()
        if r.get("reset_stats"):
            rt.reset_stats()
        rec = dict(r)
        rec["fault_rc"] = rt.set_fault(r["fault"])
        for i, x in enumerate(case_input(g, r["input"])):
            rt.set_input(i, x)
        rec["rc"] = rt.run_rc()
        rec["outputs"] = len(g.outputs) if rec["rc"] == 0 else 0
        for i in range(rec["outputs"]):
            arrays[f"{case['name']}__{len(runs)}__{i}"] = np.ascontiguousarray(rt.output(i), np.float32).view(np.uint32)
        rec["stats"] = rt.stats()
        rec["ranges"] = {}
        for p in case["protection"]:
            o = rt.observation(p["node_id"])
            rec["ranges"][str(p["node_id"])] = [f32_bits(o["observed_min"]), f32_bits(o["observed_max"]),
                                                int(o["observations"])]
        runs.append(rec)
    return runs, arrays


def ref_adapter(m) -> Adapter:
    def set_input(i, x):
        assert m.set_input(i, x) == 0

    return Adapter(m.set_fault_event, set_input, m.run_rc, m.output, m.reliability_stats, m.range_observation,
                   lambda: m.lib.spkv2_reset_range_observations(m.ctx),
                   lambda: m.lib.spkv2_reset_reliability_stats(m.ctx))


def gpu_adapter(m) -> Adapter:
    return Adapter(m.set_fault_event, m.set_input, m.run_rc, m.get_output, m.reliability_stats, m.range_observation,
                   m.reset_range_observations, m.reset_reliability_stats)
