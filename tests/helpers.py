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


def check_detections(got: list, want: list, tol: float = FP32_TOL) -> None:
    """YOLO post-processing outputs [top scores, boxes, class scores,
    indices]: the sorted top scores agree within the fp32 tolerance; anchors
    selected by both sides carry the same boxes and class scores (within
    tolerance); an anchor selected by only one side, either side, must sit
    at a near tie (its score within the tolerance of the selection
    threshold), and at most 5 of them do."""
    v, b, s, i = (np.asarray(a).reshape(a.shape) for a in got)
    wv, wb, ws, wi = (np.asarray(a) for a in want)
    k = v.size
    v, wv, i, wi = v.ravel(), wv.ravel(), i.ravel(), wi.ravel()
    b, wb = b.reshape(k, -1), wb.reshape(k, -1)
    s, ws = s.reshape(k, -1), ws.reshape(k, -1)
    assert tnorm_err(v, wv) <= tol
    scale = float(np.max(np.abs(wv)))
    pos = {int(a): n for n, a in enumerate(wi)}
    shared = [(n, pos[int(a)]) for n, a in enumerate(i) if int(a) in pos]
    for n, m in shared:
        assert float(np.abs(b[n] - wb[m]).max()) <= tol * max(1.0, float(np.abs(wb).max())), (n, b[n], wb[m])
        assert float(np.abs(s[n] - ws[m]).max()) <= tol * max(1.0, float(np.abs(ws).max())), n
    threshold = float(wv[-1])
    for n, a in enumerate(i):
        if int(a) not in pos:
            assert abs(float(v[n]) - threshold) <= tol * scale, (n, a, v[n], threshold)
    # and symmetrically: an anchor only the reference selected sits at the
    # same near tie, so the two selections differ only in how ties at the
    # threshold were broken
    mine = {int(a) for a in i}
    for m, a in enumerate(wi):
        if int(a) not in mine:
            assert abs(float(wv[m]) - threshold) <= tol * scale, (m, a, wv[m], threshold)
    assert len(shared) >= k - 5
