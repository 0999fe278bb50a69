"""Shared helpers of the parity tests."""

from __future__ import annotations

import numpy as np

# fp32 max relative error <= 1e-4 per tensor, measured
# tensor-normalized (max|a-b| / max|b|): the reference's own naive and AVX2
# conv kernels differ by ~1e-4 element-wise on small outputs.
FP32_TOL = 1e-4


def tnorm_err(a: np.ndarray, b: np.ndarray) -> float:
    a = np.asarray(a, dtype=np.float64).ravel()
    b = np.asarray(b, dtype=np.float64).ravel()
    assert a.shape == b.shape, (a.shape, b.shape)
    denom = np.max(np.abs(b))
    if denom == 0:
        return float(np.max(np.abs(a)))
    return float(np.max(np.abs(a - b)) / denom)


def rng_inputs(g, seed: int = 42, dist: str = "normal") -> list[np.ndarray]:
    from spinnv2_amd.spk.models import make_input

    return [make_input(g.tensors[t].shape, seed + i, dist) for i, t in enumerate(g.inputs)]


def run_gpu(blob: bytes, inputs: list[np.ndarray], outputs: int = 1) -> list[np.ndarray]:
    from spinnv2_amd.runtime import Model

    with Model(blob) as m:
        for i, x in enumerate(inputs):
            m.set_input(i, x)
        m.run()
        return [m.get_output(i) for i in range(outputs)]


def run_oracle(blob: bytes, inputs: list[np.ndarray]) -> list[np.ndarray]:
    from oracle.spk_exec import OracleExecutor

    return [o.ravel() for o in OracleExecutor(blob).run(*inputs)]
