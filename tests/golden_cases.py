"""Loads the golden fixtures written by tests/golden/make_golden.py.

Each fixture holds a builder call (re-run here with this repo's SPK writer),
the inputs, and the output the reference SPINNV2 C runtime produced on the
`cpu_ref` package of that graph.
"""

from __future__ import annotations

import json
from dataclasses import dataclass
from pathlib import Path

import numpy as np

GOLDEN = Path(__file__).resolve().parent / "golden"

# ops whose reference kernels are a pure selection, copy or one IEEE add per
# element: any correct restatement is bit-exact
EXACT_BUILDER_OPS = {"MaxPool", "Add", "Relu", "Resize", "Sub", "Mul", "Div", "Mod"}


@dataclass
class GoldenCase:
    name: str
    builder: str
    kwargs: dict
    inputs: list
    expected: np.ndarray        # graph output 0
    more: list | None = None    # graph outputs 1.. (multi-output ops)
    profile: str = "cpu_ref"    # the profile of the package the reference ran

    @property
    def optimized(self) -> bool:
        """The reference ran its optimized x86 kernels (Winograd, AVX2
        im2col), whose rounding a restatement of the naive kernels matches
        within the fp32 tolerance only."""
        return self.profile != "cpu_ref"

    @property
    def all_expected(self) -> list:
        return [self.expected] + list(self.more or [])

    def graph(self):
        from spinnv2_amd.spk import models

        kw = dict(self.kwargs)
        if self.builder in ("single_op", "index_op"):
            op = kw.pop("op")
            shape = kw.pop("shape")
            return getattr(models, self.builder)(op, shape, **kw)
        return getattr(models, self.builder)(**kw)

    @property
    def exact(self) -> bool:
        # index / layout ops move values without arithmetic: bit-exact
        return self.builder == "index_op" or (self.builder == "single_op" and self.kwargs["op"] in EXACT_BUILDER_OPS)


def load_cases() -> list[GoldenCase]:
    cases = []
    for p in sorted(GOLDEN.glob("*.npz")):
        with np.load(p, allow_pickle=False) as z:
            meta = json.loads(bytes(z["meta"]).decode())
            xs = [z[f"x{i}"] for i in range(len([k for k in z.files if k.startswith("x")]))]
            more = [z[f"y{o}"] for o in range(1, 1 + len([k for k in z.files if k.startswith("y") and k != "y"]))]
            cases.append(GoldenCase(p.stem, meta["builder"], meta["kwargs"], xs, z["y"], more,
                                    meta.get("profile", "cpu_ref")))
    return cases
