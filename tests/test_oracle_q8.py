"""Pins the oracle's INT8 configuration with int8 tensors between nodes
(oracle/spk_oracle.c, the oracle_q8_* functions) without the device code.

The reference runtime has no such mode (its INT8 conv keeps fp32 tensors
between nodes with zero point 0: runtime/kernels/optimized/conv/
conv_int8.c:121-210, compiler/quantization/calibrate.py:16), so nothing can
be checked against reference outputs.  Instead:
  * the round-half-away shift against exact rationals (fractions.Fraction),
    at constructed ties of both signs and at random points;
  * the fixed-point multipliers against the exact rational scale ratios of
    the float32 scales, and one requantization against exact rational
    arithmetic (the bias, residual, Relu clamp and saturation included);
  * the conv accumulators against int64 brute force in numpy on an input
    padded with the zero point, i.e. through the zero-point identity
    sum w (x - z) = sum w x' - z sum w (x' padded with z), a different
    algorithm from the oracle's skipped taps;
  * quantize, MaxPool and the dequantizing mean against closed forms.
"""

from __future__ import annotations

import ctypes
from fractions import Fraction

import numpy as np
import pytest

from oracle.spk_exec import _lib

I64, I32, F32, VP = ctypes.c_int64, ctypes.c_int32, ctypes.c_float, ctypes.c_void_p


@pytest.fixture(scope="module")
def lib():
    lib = _lib()
    lib.oracle_q8_round_shift.restype = I64
    lib.oracle_q8_round_shift.argtypes = [I64, ctypes.c_int]
    lib.oracle_q8_requant_one.restype = ctypes.c_int
    lib.oracle_q8_requant_one.argtypes = [I32, I32, I32, I32, I32, ctypes.c_int, ctypes.c_int, ctypes.c_int]
    lib.oracle_q8_requant_params.restype = ctypes.c_int
    lib.oracle_q8_requant_params.argtypes = [F32, VP, F32, F32, VP, ctypes.c_int, VP, VP, VP, VP]
    return lib


def _p(a):
    return a.ctypes.data_as(VP) if a is not None else None


def rha(q: Fraction) -> int:
    """Exact rational rounded to nearest, ties away from zero."""
    fl = q.numerator // q.denominator
    frac = q - fl
    if frac > Fraction(1, 2) or (frac == Fraction(1, 2) and q > 0):
        return fl + 1
    return fl


def test_round_shift_ties_and_random(lib):
    rng = np.random.default_rng(3)
    for s in (1, 2, 5, 17, 31, 40, 62):
        half = 1 << (s - 1)
        for k in (0, 1, 2, 7, 1000):
            t = (2 * k + 1) * half  # exactly k + 0.5 after the shift
            if t >= 1 << 62:
                continue
            assert lib.oracle_q8_round_shift(t, s) == k + 1
            assert lib.oracle_q8_round_shift(-t, s) == -(k + 1)
            assert lib.oracle_q8_round_shift(t - 1, s) == k  # just below the tie
            assert lib.oracle_q8_round_shift(-t + 1, s) == -k
        for t in rng.integers(-(1 << 61), 1 << 61, 200):
            assert lib.oracle_q8_round_shift(int(t), s) == rha(Fraction(int(t), 1 << s))


def _params(lib, sx, sw, sy, sr, bias):
    M = len(sw)
    sw = np.asarray(sw, np.float32)
    out = [np.zeros(M, np.int32) for _ in range(4)]
    b = None if bias is None else np.asarray(bias, np.float32)
    rc = lib.oracle_q8_requant_params(sx, _p(sw), sy, sr, _p(b), M, *(_p(o) for o in out))
    return rc, out


def test_requant_params_against_exact_ratios(lib):
    rng = np.random.default_rng(5)
    for _ in range(50):
        sx, sy, sr = (float(np.float32(v)) for v in rng.uniform(1e-3, 0.2, 3))
        sw = rng.uniform(1e-4, 5e-2, 16).astype(np.float32)
        bias = rng.normal(0, 0.5, 16).astype(np.float32)
        has_res = rng.random() < 0.5
        rc, (bq, m1, m2, sh) = _params(lib, sx, sw, sy, sr if has_res else 0.0, bias)
        assert rc == 0
        for m in range(16):
            S = int(sh[m])
            r1 = Fraction(sx) * Fraction(float(sw[m])) / Fraction(sy)
            r2 = Fraction(sr) / Fraction(sy) if has_res else Fraction(0)
            # nearest integers to the exact scaled ratios, the larger in [2^29, 2^31)
            assert abs(Fraction(int(m1[m])) - r1 * (1 << S)) <= Fraction(1, 2)
            assert abs(Fraction(int(m2[m])) - r2 * (1 << S)) <= Fraction(1, 2)
            assert (1 << 29) <= max(int(m1[m]), int(m2[m])) < (1 << 31)
            # bias in accumulator units, rounded half away (float64 quotient:
            # skip values within 1e-6 of a tie)
            exact = Fraction(float(bias[m])) / (Fraction(sx) * Fraction(float(sw[m])))
            if abs(exact - exact.numerator // exact.denominator - Fraction(1, 2)) > Fraction(1, 10 ** 6):
                assert int(bq[m]) == rha(exact)


def test_requant_one_exact_rationals(lib):
    rng = np.random.default_rng(9)
    for _ in range(2000):
        S = int(rng.integers(20, 45))
        m1 = int(rng.integers(1 << 29, 1 << 31))
        m2 = int(rng.integers(0, 1 << 31))
        acc = int(rng.integers(-(1 << 26), 1 << 26))
        bq = int(rng.integers(-(1 << 20), 1 << 20))
        r = int(rng.integers(-255, 256))
        zy = int(rng.integers(-128, 128))
        relu = int(rng.integers(0, 2))
        v = rha(Fraction((acc + bq) * m1 + r * m2, 1 << S)) + zy
        if relu:
            v = max(v, zy)
        want = max(-128, min(127, v))
        assert lib.oracle_q8_requant_one(acc, bq, m1, m2, S, r, zy, relu) == want
    # constructed ties: multiplier 1/2 (m1 = 2^(S-1)), odd sums land on .5
    S = 10
    for a in (-7, -3, -1, 1, 3, 5, 101):
        want = (abs(a) + 1) // 2 * (1 if a > 0 else -1)
        assert lib.oracle_q8_requant_one(a, 0, 1 << (S - 1), 0, S, 0, 0, 0) == max(-128, min(127, want))
    # the Relu clamp holds at the zero point, saturation at both ends
    assert lib.oracle_q8_requant_one(-1000, 0, 1 << 30, 0, 30, 0, -5, 1) == -5
    assert lib.oracle_q8_requant_one(-1000, 0, 1 << 30, 0, 30, 0, -5, 0) == -128
    assert lib.oracle_q8_requant_one(10 ** 6, 0, 1 << 30, 0, 30, 0, 0, 0) == 127


def _conv_case(rng, N, C, H, W, M, k, s, p, d, res):
    x = rng.integers(-128, 128, (N, C, H, W)).astype(np.int8)
    w = rng.integers(-128, 128, (M, C, k, k)).astype(np.int8)
    zx, zr, zy = (int(v) for v in rng.integers(-128, 128, 3))
    OH = (H + 2 * p - d * (k - 1) - 1) // s + 1
    OW = (W + 2 * p - d * (k - 1) - 1) // s + 1
    r = rng.integers(-128, 128, (N, M, OH, OW)).astype(np.int8) if res else None
    return x, w, zx, zr, zy, r, OH, OW


@pytest.mark.parametrize("case", [(2, 3, 5, 4, 4, 3, 2, 1, 1, True), (1, 5, 6, 6, 3, 3, 1, 1, 1, False),
                                  (2, 4, 7, 5, 2, 3, 1, 2, 2, True), (1, 16, 4, 4, 8, 1, 1, 0, 1, True),
                                  (1, 3, 9, 9, 2, 7, 2, 3, 1, False)])
def test_conv_accumulators_zero_point_identity(lib, case):
    N, C, H, W, M, k, s, p, d, res = case
    rng = np.random.default_rng(sum(case))
    x, w, zx, zr, zy, r, OH, OW = _conv_case(rng, *case)
    sx, sy, sr = 0.05, 0.07, 0.09
    sw = rng.uniform(1e-3, 1e-2, M).astype(np.float32)
    bias = rng.normal(0, 0.3, M).astype(np.float32)
    rc, (bq, m1, m2, sh) = _params(lib, sx, sw, sy, sr if res else 0.0, bias)
    assert rc == 0
    y = np.zeros((N, M, OH, OW), np.int8)
    acc = np.zeros((N, M, OH, OW), np.int32)
    lib.oracle_q8_conv(_p(x), zx, _p(w), _p(bq), _p(m1), _p(m2), _p(sh), _p(r), zr, zy, 1, _p(y), _p(acc),
                       N, C, H, W, M, k, k, OH, OW, s, s, p, p, d, d)
    # brute force: the input padded with its zero point (real zero), all taps
    xp = np.pad(x.astype(np.int64), ((0, 0), (0, 0), (p, p), (p, p)), constant_values=zx)
    raw = np.zeros((N, M, OH, OW), np.int64)
    for kh in range(k):
        for kw in range(k):
            patch = xp[:, :, kh * d: kh * d + s * (OH - 1) + 1: s, kw * d: kw * d + s * (OW - 1) + 1: s]
            raw += np.einsum("nchw,mc->nmhw", patch, w[:, :, kh, kw].astype(np.int64))
    want_acc = raw - zx * w.astype(np.int64).sum(axis=(1, 2, 3))[None, :, None, None]
    np.testing.assert_array_equal(acc, want_acc)
    # every output through exact rational requantization
    for idx in np.ndindex(N, M, OH, OW):
        m = idx[1]
        rd = int(r[idx]) - zr if res else 0
        v = rha(Fraction((int(want_acc[idx]) + int(bq[m])) * int(m1[m]) + rd * int(m2[m]), 1 << int(sh[m]))) + zy
        assert int(y[idx]) == max(-128, min(127, max(v, zy))), idx


def test_quantize_closed_form(lib):
    s, z = 0.25, 3  # 1/s = 4 exactly: x * inv is exact
    x = np.array([0.125, -0.125, 0.375, -0.375, 0.0, 1e9, -1e9, np.nan, 31.9, -32.1], np.float32)
    q = np.zeros(x.size, np.int8)
    lib.oracle_q8_quantize(_p(x), _p(q), ctypes.c_size_t(x.size), F32(s), z)
    # 0.5 -> 1, -0.5 -> -1, 1.5 -> 2, -1.5 -> -2 (half away), + z, saturated, NaN -> z
    assert q.tolist() == [4, 2, 5, 1, 3, 127, -128, 3, 127, -125]


def test_maxpool_and_mean_closed_forms(lib):
    rng = np.random.default_rng(1)
    x = rng.integers(-128, 128, (2, 3, 7, 6)).astype(np.int8)
    OH, OW = 4, 3
    y = np.zeros((2, 3, OH, OW), np.int8)
    lib.oracle_q8_maxpool(_p(x), _p(y), 2, 3, 7, 6, OH, OW, 3, 3, 2, 2, 1, 1)
    xp = np.pad(x.astype(np.int16), ((0, 0), (0, 0), (1, 1), (1, 1)), constant_values=-1000)
    want = np.full((2, 3, OH, OW), -1000, np.int16)
    for kh in range(3):
        for kw in range(3):
            want = np.maximum(want, xp[:, :, kh: kh + 2 * (OH - 1) + 1: 2, kw: kw + 2 * (OW - 1) + 1: 2])
    np.testing.assert_array_equal(y, want)
    m = np.zeros(6, np.float32)
    s, z = 0.037, -11
    lib.oracle_q8_plane_mean(_p(x), _p(m), ctypes.c_size_t(6), 42, F32(s), z)
    for p_, v in enumerate(m):
        exact = Fraction(int(x.reshape(6, 42)[p_].astype(np.int64).sum()) - 42 * z) * Fraction(float(np.float32(s))) / 42
        # one float32 rounding of a value within two float64 roundings of exact
        assert abs(Fraction(float(v)) - exact) <= abs(exact) * Fraction(1, 1 << 23) + Fraction(1, 10 ** 30)


def test_asymmetric_params_map_range_ends():
    from spinnv2_amd.spk.quantize import asymmetric_params

    for lo, hi in [(-1.3, 4.2), (0.0, 6.0), (-3.0, -0.5), (-0.01, 100.0), (0.0, 0.0)]:
        s, z = asymmetric_params(lo, hi)
        assert -128 <= z <= 127
        lo0, hi0 = min(lo, 0.0), max(hi, 0.0)
        if hi0 > lo0:
            # the ends of the (zero-widened) range land within half a step of
            # the int8 ends; real 0 is exactly the zero point
            assert abs(lo0 / s + z - (-128)) <= 0.5 + 1e-6 or z == 127
            assert abs(hi0 / s + z - 127) <= 1.0 + 1e-6
    assert asymmetric_params(0.0, 6.0)[1] == -128  # a Relu output: [0, max] -> [-128, 127]


def test_int8_tensor_plan_resnet_and_fallback():
    from spinnv2_amd.spk import models
    from spinnv2_amd.spk.graph import Graph
    from spinnv2_amd.spk.passes import run_default_pipeline
    from spinnv2_amd.spk.quantize import int8_tensor_plan

    g = models.resnet(50, 1, image=32, classes=10)
    cand, convs = int8_tensor_plan(g)
    assert len(convs) == 53 and len(cand) == 54  # 53 conv outputs and the stem MaxPool's
    # a conv whose output feeds a Gemm stays fp32, and so does the tensor
    # feeding it (its reader does not run in the mode)
    p = models.Params(3)
    h = Graph("t")
    x = h.input("x", [1, 3, 8, 8])
    a = h.relu(h.conv(x, p.he((8, 3, 3, 3)), p.normal(8, 0.01), pad=1))
    b = h.relu(h.conv(a, p.he((8, 8, 1, 1)), p.normal(8, 0.01)))
    c = h.gemm(h.flatten(b, 1), p.he((512, 10)))
    h.mark_output(c)
    run_default_pipeline(h)
    cand, convs = int8_tensor_plan(h)
    assert cand == set() and convs == []
    # a SiLU conv keeps its fp32 output (the requantizing epilogue clamps
    # Relu only), so the tensor it reads stays fp32 too; the conv after it
    # quantizes that fp32 input on load
    s = Graph("silu")
    x = s.input("x", [1, 3, 8, 8])
    a = s.relu(s.conv(x, p.he((8, 3, 3, 3)), p.normal(8, 0.01), pad=1))
    b = s.silu(s.conv(a, p.he((8, 8, 3, 3)), p.normal(8, 0.01), pad=1))
    c = s.relu(s.conv(b, p.he((16, 8, 1, 1)), p.normal(16, 0.01)))
    s.mark_output(s.flatten(s.reduce_mean(c, [2, 3], keepdims=1), 1))
    run_default_pipeline(s)
    convs_all = [n for n in s.nodes if n.op_type == "Conv"]
    assert [n.attrs.get("fused_activation") for n in convs_all] == ["Relu", "Silu", "Relu"]
    cand, convs = int8_tensor_plan(s)
    assert convs == [convs_all[2]] and cand == {convs_all[2].outputs[0]}


def test_oracle_q8_resnet_tracks_fp32():
    """End to end on a small ResNet-50: the mode's logits stay near the fp32
    network's (a loose sanity bound; the parity bars are the tests above)."""
    from oracle.spk_exec import OracleExecutor
    from spinnv2_amd.spk import models, write_spk
    from spinnv2_amd.spk.quantize import forward_fp32, quantize_int8_activations

    g = models.resnet(50, 1, image=64, classes=10)
    ref_g = models.resnet(50, 1, image=64, classes=10)
    samples = [models.make_input(g.tensors[g.inputs[0]].shape, 1000 + i) for i in range(4)]
    qp = quantize_int8_activations(g, samples)
    blob = write_spk(g, "mi355x", quant_params=qp)
    x = models.make_input(g.tensors[g.inputs[0]].shape, 42)
    got = OracleExecutor(blob).run(x)[0].ravel()
    want = forward_fp32(ref_g, [x], {ref_g.outputs[0]})[ref_g.outputs[0]].ravel()
    assert np.abs(got - want).max() <= 0.1 * np.abs(want).max()


def test_q8_package_records_and_loader():
    """The mode's package: int8 activation tensors (dtype 2, role
    activation) of numel bytes in the memory plan, a per-tensor record with
    a zero point for each, and the runtime loader accepts it."""
    import ctypes as ct

    from oracle.spk_exec import Package
    from spinnv2_amd.runtime import load_library
    from spinnv2_amd.spk import models, write_spk

    g = models.resnet(50, 1, image=32, classes=10)
    samples = [models.make_input(g.tensors[g.inputs[0]].shape, 1000 + i) for i in range(2)]
    from spinnv2_amd.spk.quantize import quantize_int8_activations

    blob = write_spk(g, "mi355x", quant_params=quantize_int8_activations(g, samples))
    pkg = Package(blob)
    q8 = [t for t in pkg.tensors if t.dtype == 2 and t.role == 4]
    assert len(q8) == 54
    for t in q8:
        assert t.size == int(np.prod(t.shape))
        assert len(pkg.quant[t.id]) == 1 and -128 <= int(pkg.zero_points[t.id][0]) <= 127
    lib = load_library()
    buf = ct.create_string_buffer(blob, len(blob))
    ctx = ct.c_void_p()
    assert lib.spkv2_load_memory(buf, len(blob), ct.byref(ctx)) == 0
    lib.spkv2_free(ctx)


def test_device_requant_math_equals_oracle(tmp_path, lib):
    """spinnv2_amd/csrc/kernels/q8_math.hpp (the device epilogue's
    requantization, built here for the host with g++): the general form and
    the high-word form (shift 33..55, output zero point folded into the
    rounding constant) equal the oracle's single rounding on
    random values and on constructed ties of both signs, where the high-word
    form's borrow rule decides."""
    import subprocess
    from pathlib import Path

    hdr = Path(__file__).resolve().parent.parent / "spinnv2_amd" / "csrc" / "kernels"
    src = tmp_path / "shim.cpp"
    src.write_text('#include "q8_math.hpp"\n'
                   'extern "C" int rq(int a, int c, int m1, int m2, int sh, int rd, int zy, int lo) '
                   '{ return spk::kern::q8_requant(a, c, m1, m2, sh, rd, zy, lo); }\n'
                   'extern "C" int rq_hi(int a, int c, int m1, int m2, int k, int rd, int zy, int lo) '
                   '{ return spk::kern::q8_requant_hi(a, c, m1, m2, (1 << (k - 1)) + zy * (1 << k), k, rd, lo, '
                   'spk::kern::q8_clamp); }\n')
    so = tmp_path / "shim.so"
    subprocess.run(["g++", "-std=c++17", "-O2", "-shared", "-fPIC", f"-I{hdr}", str(src), "-o", str(so)], check=True)
    shim = ctypes.CDLL(str(so))
    for f in (shim.rq, shim.rq_hi):
        f.restype = ctypes.c_int
        f.argtypes = [ctypes.c_int] * 8
    rng = np.random.default_rng(21)
    cases = []
    for _ in range(20000):
        S = int(rng.integers(33, 56))
        cases.append((int(rng.integers(-(1 << 27), 1 << 27)), int(rng.integers(-(1 << 29), 1 << 29)),
                      int(rng.integers(1 << 29, 1 << 31)), int(rng.integers(0, 1 << 31)), S,
                      int(rng.integers(-255, 256)), int(rng.integers(-128, 128)), int(rng.integers(0, 2))))
    # ties: t = (2j + 1) 2^(S-1) exactly, both signs, with and without a low word
    for S in (33, 34, 40, 47, 55):
        for j in (0, 1, 5, 100):
            for sign in (1, -1):
                # m1 = 2^(S-1-e) times an odd A gives t = A 2^(S-1-e); choose A = (2j+1) 2^e
                m1 = 1 << 30
                e = S - 1 - 30
                if e < 0:
                    continue
                A = sign * (2 * j + 1) * (1 << e)
                cases.append((A, 0, m1, 0, S, 0, 0, 0))
                cases.append((A + sign, 0, m1, 0, S, 0, 0, 0))  # just past the tie
                cases.append((A - sign, 0, m1, 0, S, 0, 0, 0))  # just before it
    for acc, c, m1, m2, S, rd, zy, relu in cases:
        lo = zy if relu else -128
        want = lib.oracle_q8_requant_one(acc, c, m1, m2, S, rd, zy, relu)
        assert shim.rq(acc, c, m1, m2, S, rd, zy, lo) == want, (acc, c, m1, m2, S, rd, zy, relu)
        assert shim.rq_hi(acc, c, m1, m2, S - 32, rd, zy, lo) == want, (acc, c, m1, m2, S, rd, zy, relu)
