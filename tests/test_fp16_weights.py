"""FP16-weight packages (the reference's --fp16-weights, compiler/passes/
convert_fp16.py:11-25): rank >= 2 fp32 weights stored as IEEE half, widened
back to fp32 by the runtime (reference runtime/kernels/optimized/conv/
conv.c:961-978 and mm/gemm.c:150-162; this runtime does it once at load).

Half -> float widening is exact, so a half-weight package must compute
exactly what the fp32 package computes with its weights rounded to half
first.  That closed form pins the oracle and the GPU runtime without the
reference (whose x86 build returns -99 for half weights: its promotion is
compiled only for ARM).
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest

from spinnv2_amd.spk import format as F
from spinnv2_amd.spk import models, write_spk
from spinnv2_amd.spk.passes import convert_weights_fp16

from .helpers import FP32_TOL, rng_inputs, run_gpu, run_oracle, tnorm_err

BUILDS = {
    "lenet": lambda: models.lenet(),
    "resnet18_32px": lambda: models.resnet(18, batch=2, image=32, classes=10),
    "yolov10n_160": lambda: models.yolo_v10n(image=160, topk=50),
}


def rounded_fp32(g):
    """The same graph with the half-stored weights rounded to half but kept fp32."""
    for t in g.tensors:
        if t.role == "weight" and t.dtype == "fp32" and t.data is not None and len(t.shape) >= 2:
            t.data = np.asarray(t.data, np.float32).astype(np.float16).astype(np.float32)
    return g


def pair(name):
    g16 = BUILDS[name]()
    n = convert_weights_fp16(g16)
    assert n > 0
    return g16, rounded_fp32(BUILDS[name]())


def test_widening_is_exact_for_every_half(lib):
    h = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    out = np.empty(h.size, dtype=np.uint32)
    lib.spkv2_mi355x_fp16_to_fp32(h.ctypes.data_as(ctypes.c_void_p), out.ctypes.data_as(ctypes.c_void_p), h.size)
    want = h.view(np.float16).astype(np.float32).view(np.uint32)
    finite = ~np.isnan(h.view(np.float16))
    np.testing.assert_array_equal(out[finite], want[finite])
    # NaNs: sign kept, payload in the high mantissa bits, still NaN
    nan = ~finite
    assert np.isnan(out[nan].view(np.float32)).all()
    np.testing.assert_array_equal(out[nan], ((h[nan].astype(np.uint32) & 0x8000) << 16) | 0x7F800000
                                  | ((h[nan].astype(np.uint32) & 0x3FF) << 13))


def test_conversion_pass_follows_the_reference():
    g = models.lenet()
    ranks = {t.id: len(t.shape) for t in g.tensors if t.role == "weight"}
    before = {t.id: t.data.copy() for t in g.tensors if t.role == "weight"}
    n = convert_weights_fp16(g)
    assert n == sum(r >= 2 for r in ranks.values())
    assert convert_weights_fp16(g) == 0      # idempotent
    blob = write_spk(g, "mi355x")
    hdr = F.HEADER.unpack_from(blob, 0)
    secs = {s[0]: s for s in (F.SECTION.unpack_from(blob, hdr[4] + i * F.SECTION.size) for i in range(hdr[5]))}
    toff, woff = secs[F.SECTION_TENSOR_TABLE][2], secs[F.SECTION_WEIGHTS][2]
    for tid, rank in ranks.items():
        rec = F.TENSOR.unpack_from(blob, toff + tid * F.TENSOR.size)
        dtype, size, off = rec[1], rec[13], rec[14]
        numel = before[tid].size
        if rank >= 2:
            assert (dtype, size) == (3, 2 * numel)
            stored = np.frombuffer(blob, "<f2", numel, woff + off)
            np.testing.assert_array_equal(stored, before[tid].ravel().astype(np.float16))
        else:
            assert (dtype, size) == (1, 4 * numel)


@pytest.mark.parametrize("name", ["lenet", "resnet18_32px"])
def test_oracle_half_weights_equal_rounded_fp32(name):
    g16, g32 = pair(name)
    xs = rng_inputs(g32, seed=5)
    a = run_oracle(write_spk(g16, "mi355x"), xs)
    b = run_oracle(write_spk(g32, "mi355x"), xs)
    for u, v in zip(a, b):
        np.testing.assert_array_equal(u.view(np.uint32), v.view(np.uint32))


@pytest.mark.gpu
@pytest.mark.parametrize("name", list(BUILDS))
def test_gpu_half_weights_equal_rounded_fp32(gpu, name):
    print(f"[fp16 weights] {name}", flush=True)
    g16, g32 = pair(name)
    xs = rng_inputs(g32, seed=5)
    n_out = len(g32.outputs)
    b = run_gpu(write_spk(g32, "mi355x"), xs, outputs=n_out)
    a = run_gpu(write_spk(g16, "mi355x"), xs, outputs=n_out)    # same shapes: same tuned tiles
    for u, v in zip(a, b):
        np.testing.assert_array_equal(u.view(np.uint32), v.view(np.uint32))
    if name != "yolov10n_160":
        want = run_oracle(write_spk(g16, "mi355x"), xs)[0]
        assert tnorm_err(a[0].ravel(), want) <= FP32_TOL
