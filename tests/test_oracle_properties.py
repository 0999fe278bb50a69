"""Pins the CPU oracle (oracle/liboracle.so) without the reference runtime:
the reference's own C known-answer tests, closed forms brute-forced in
float64 / int64 / exact rationals, and invariants.  No GPU.

Each check is chosen so that a plausible restatement mistake fails it:
non-square, non-symmetric shapes and kernels (a transposed index or
swapped kh/kw), asymmetric padding and dilation (a wrong sign or offset),
residual before activation (wrong order), and explicit rounding ties for
the INT8 quantizer (wrong rounding rule or chunk boundary).
"""

from __future__ import annotations

import ctypes
from fractions import Fraction

import numpy as np
import pytest

from oracle.spk_exec import _lib

LIB = _lib()
vp = ctypes.c_void_p


def P(a):
    return a.ctypes.data_as(vp) if a is not None else None


def conv_oracle(x, w, b=None, r=None, stride=(1, 1), pad=(0, 0), dil=(1, 1), group=1, act=0):
    N, C, H, W = x.shape
    M, _, KH, KW = w.shape
    OH = (H + 2 * pad[0] - dil[0] * (KH - 1) - 1) // stride[0] + 1
    OW = (W + 2 * pad[1] - dil[1] * (KW - 1) - 1) // stride[1] + 1
    y = np.zeros((N, M, OH, OW), np.float32)
    rc = LIB.oracle_conv2d_f32(P(x), P(w), P(b), P(r), P(y), N, C, H, W, M, KH, KW, OH, OW, stride[0], stride[1],
                               pad[0], pad[1], dil[0], dil[1], group, act)
    assert rc == 0
    return y


def conv_brute64(x, w, b, r, stride, pad, dil, group, act):
    """float64 direct sum of the convolution definition (zero padding)."""
    x = x.astype(np.float64)
    w = w.astype(np.float64)
    N, C, H, W = x.shape
    M, Cg, KH, KW = w.shape
    OH = (H + 2 * pad[0] - dil[0] * (KH - 1) - 1) // stride[0] + 1
    OW = (W + 2 * pad[1] - dil[1] * (KW - 1) - 1) // stride[1] + 1
    xp = np.zeros((N, C, H + 2 * pad[0], W + 2 * pad[1]))
    xp[:, :, pad[0]:pad[0] + H, pad[1]:pad[1] + W] = x
    y = np.zeros((N, M, OH, OW))
    Mg = M // group
    for m in range(M):
        c0 = (m // Mg) * Cg
        for kh in range(KH):
            for kw in range(KW):
                patch = xp[:, c0:c0 + Cg, kh * dil[0]: kh * dil[0] + stride[0] * (OH - 1) + 1: stride[0],
                           kw * dil[1]: kw * dil[1] + stride[1] * (OW - 1) + 1: stride[1]]
                y[:, m] += np.einsum("nchw,c->nhw", patch, w[m, :, kh, kw])
        if b is not None:
            y[:, m] += b[m]
    if r is not None:
        y += r
    if act == 1:
        y = np.maximum(y, 0)
    elif act == 2:
        y = y / (1 + np.exp(-y))
    return y


RNG = np.random.default_rng(2024)

CONV_SHAPES = [
    # (N, C, H, W, M, KH, KW, stride, pad, dil, group, act, bias, res)
    (1, 3, 7, 9, 4, 3, 2, (1, 1), (1, 0), (1, 1), 1, 0, True, False),   # non-square kernel, asymmetric pad
    (2, 4, 10, 8, 6, 3, 3, (2, 1), (1, 2), (1, 1), 1, 1, True, True),   # strides differ per axis, residual+relu
    (1, 5, 9, 9, 3, 3, 3, (1, 1), (2, 2), (2, 2), 1, 0, False, False),  # dilation 2
    (1, 6, 6, 7, 9, 1, 3, (1, 2), (0, 1), (1, 1), 3, 2, True, False),   # groups, SiLU
    (2, 8, 5, 5, 8, 3, 3, (1, 1), (1, 1), (1, 1), 8, 1, True, False),   # depthwise
]


@pytest.mark.parametrize("shape", CONV_SHAPES)
def test_conv_matches_float64_definition(shape):
    N, C, H, W, M, KH, KW, stride, pad, dil, group, act, has_b, has_r = shape
    x = RNG.standard_normal((N, C, H, W)).astype(np.float32)
    w = RNG.standard_normal((M, C // group, KH, KW)).astype(np.float32)
    b = RNG.standard_normal(M).astype(np.float32) if has_b else None
    y64 = conv_brute64(x, w, b, None, stride, pad, dil, group, 0)
    r = RNG.standard_normal(y64.shape).astype(np.float32) if has_r else None
    got = conv_oracle(x, w, b, r, stride, pad, dil, group, act)
    want = conv_brute64(x, w, b, r, stride, pad, dil, group, act)
    assert got.shape == want.shape
    np.testing.assert_allclose(got, want, rtol=0, atol=1e-5 * max(1.0, np.abs(want).max()))


def test_conv_residual_is_added_before_activation():
    # bias -3, residual +5: Relu(conv + bias + res) differs from Relu(conv + bias) + res
    x = np.zeros((1, 1, 3, 3), np.float32)
    w = np.zeros((1, 1, 1, 1), np.float32)
    b = np.array([-3.0], np.float32)
    r = np.full((1, 1, 3, 3), 5.0, np.float32)
    np.testing.assert_array_equal(conv_oracle(x, w, b, r, act=1), np.full((1, 1, 3, 3), 2.0, np.float32))


def test_conv_batch_invariance_bitwise():
    x = RNG.standard_normal((3, 6, 9, 9)).astype(np.float32)
    w = RNG.standard_normal((5, 6, 3, 3)).astype(np.float32)
    b = RNG.standard_normal(5).astype(np.float32)
    full = conv_oracle(x, w, b, pad=(1, 1))
    for i in range(3):
        one = conv_oracle(np.ascontiguousarray(x[i:i + 1]), w, b, pad=(1, 1))
        np.testing.assert_array_equal(full[i:i + 1].view(np.uint32), one.view(np.uint32))


def test_conv_linearity_power_of_two_exact():
    x = RNG.standard_normal((1, 4, 6, 6)).astype(np.float32)
    w = RNG.standard_normal((3, 4, 3, 3)).astype(np.float32)
    y1 = conv_oracle(x, w, pad=(1, 1))
    y2 = conv_oracle(x, 4 * w, pad=(1, 1))
    np.testing.assert_array_equal(4 * y1, y2)


@pytest.mark.parametrize("trans_a,trans_b,alpha", [(0, 0, 1.0), (0, 1, 0.5), (1, 0, 2.0), (1, 1, 1.0)])
def test_gemm_matches_float64(trans_a, trans_b, alpha):
    rows, K, nout = 5, 37, 11
    a = RNG.standard_normal((K, rows) if trans_a else (rows, K)).astype(np.float32)
    b = RNG.standard_normal((nout, K) if trans_b else (K, nout)).astype(np.float32)
    c = RNG.standard_normal(nout).astype(np.float32)
    y = np.zeros((rows, nout), np.float32)
    LIB.oracle_gemm_f32(P(a), P(b), P(c), P(y), rows, K, nout, trans_a, trans_b, ctypes.c_float(alpha))
    A = a.T if trans_a else a
    B = b.T if trans_b else b
    want = alpha * (A.astype(np.float64) @ B.astype(np.float64)) + c
    np.testing.assert_allclose(y, want, rtol=0, atol=1e-5 * np.abs(want).max())


# ------------------------------------------------------------ reference KATs

def test_kat_maxpool():
    """reference runtime/tests/test_kernel_maxpool.c:24-44 and 66-86."""
    x = np.arange(1, 17, dtype=np.float32).reshape(1, 1, 4, 4)
    y = np.zeros((1, 1, 2, 2), np.float32)
    LIB.oracle_maxpool_f32(P(x), P(y), 1, 1, 4, 4, 2, 2, 2, 2, 2, 2, 0, 0)
    assert y.ravel().tolist() == [6.0, 8.0, 14.0, 16.0]
    x = np.array([-5, -3, -1, -7, -2, -4, -6, -8, -9, -1, -3, -5, -7, -2, -4, -6], np.float32).reshape(1, 1, 4, 4)
    LIB.oracle_maxpool_f32(P(x), P(y), 1, 1, 4, 4, 2, 2, 2, 2, 2, 2, 0, 0)
    assert y.ravel().tolist() == [-2.0, -1.0, -1.0, -3.0]


def _binary(op, a, b, y_shape, act=0):
    y = np.zeros(y_shape, np.float32)
    sa = np.array(a.shape, np.uint32)
    sb = np.array(b.shape, np.uint32)
    sy = np.array(y_shape, np.uint32)
    rc = LIB.oracle_binary_f32(op, P(a), P(sa), a.ndim, P(b), P(sb), b.ndim, P(y), P(sy), len(y_shape), act)
    assert rc == 0
    return y


def test_kat_add():
    """reference runtime/tests/test_kernel_add.c:17-36 (same shape) and
    54-73 (b broadcast over [1,4,1,1])."""
    a = np.arange(16, dtype=np.float32).reshape(1, 4, 2, 2)
    b = (np.arange(16, dtype=np.float32) * 10).reshape(1, 4, 2, 2)
    np.testing.assert_array_equal(_binary(1, a, b, (1, 4, 2, 2)), a + b)
    b = (100.0 * np.arange(1, 5, dtype=np.float32)).reshape(1, 4, 1, 1)
    np.testing.assert_array_equal(_binary(1, a, b, (1, 4, 2, 2)), a + b)


def test_kat_relu():
    """reference runtime/tests/test_kernel_relu.c:13-31."""
    x = np.array([-3.0, -1.0, -0.5, 0.0, 0.5, 1.0, 2.0, 100.0], np.float32)
    y = np.zeros_like(x)
    LIB.oracle_relu_f32(P(x), P(y), ctypes.c_size_t(8))
    assert y.tolist() == [0.0, 0.0, 0.0, 0.0, 0.5, 1.0, 2.0, 100.0]


@pytest.mark.parametrize("x", [[1.0, 2.0, 3.0, 4.0], [1000.0, 1001.0, 1002.0, 1003.0]])
def test_kat_softmax(x):
    """reference runtime/tests/test_kernel_softmax.c:17-37 and 50-66: in
    (0, 1), sums to 1, monotone, finite for large inputs; plus the closed
    form exp(x - max) / sum."""
    x = np.array(x, np.float32)
    y = np.zeros_like(x)
    LIB.oracle_softmax_f32(P(x), P(y), ctypes.c_size_t(1), ctypes.c_size_t(4), ctypes.c_size_t(1))
    assert np.all(np.isfinite(y)) and np.all(y > 0) and np.all(y < 1)
    assert abs(float(y.sum()) - 1.0) < 1e-5
    assert y[3] > y[2] > y[1] > y[0]
    e = np.exp(x.astype(np.float64) - x.max())
    np.testing.assert_allclose(y, e / e.sum(), rtol=1e-6)


def test_softmax_inner_axis():
    x = RNG.standard_normal((2, 5, 3)).astype(np.float32)
    y = np.zeros_like(x)
    LIB.oracle_softmax_f32(P(x), P(y), ctypes.c_size_t(2), ctypes.c_size_t(5), ctypes.c_size_t(3))
    e = np.exp(x.astype(np.float64) - x.max(axis=1, keepdims=True))
    np.testing.assert_allclose(y, e / e.sum(axis=1, keepdims=True), rtol=1e-6)


def test_resize_nearest_is_replication():
    x = RNG.standard_normal((2, 3, 4, 5)).astype(np.float32)
    y = np.zeros((2, 3, 8, 10), np.float32)
    LIB.oracle_resize_nearest_f32(P(x), P(y), 2, 3, 4, 5, 8, 10)
    np.testing.assert_array_equal(y, x.repeat(2, axis=2).repeat(2, axis=3))


def test_reduce_mean_and_max():
    x = RNG.standard_normal((2, 3, 4, 5)).astype(np.float32)
    shp = np.array(x.shape, np.uint32)
    y = np.zeros((2, 3, 1, 1), np.float32)
    LIB.oracle_reduce_f32(P(x), P(shp), 4, 0b1100, 0, P(y))
    np.testing.assert_allclose(y, x.astype(np.float64).mean(axis=(2, 3), keepdims=True), rtol=1e-5, atol=1e-6)
    ym = np.zeros((2, 1, 4, 5), np.float32)
    LIB.oracle_reduce_f32(P(x), P(shp), 4, 0b0010, 1, P(ym))
    np.testing.assert_array_equal(ym, x.max(axis=1, keepdims=True))


# -------------------------------------------------------------------- INT8

def quantize(x, scale):
    q = np.zeros(x.size, np.int8)
    LIB.oracle_quantize_act(P(x), P(q), ctypes.c_size_t(x.size), ctypes.c_float(scale))
    return q


def test_quantize_ties_follow_chunk_rule():
    """reference optimized/conv/conv_int8.c:26-55: the 16-wide loop rounds
    half to even (vcvtnq), the scalar tail rounds half away (roundf)."""
    ties = np.array([0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 3.5, -3.5], np.float32)
    x = np.concatenate([ties, ties, ties[:5]])  # 16 in the vector body, 5 in the tail
    q = quantize(x, 1.0)
    assert q[:8].tolist() == [0, 2, 2, 0, -2, -2, 4, -4]
    assert q[8:16].tolist() == [0, 2, 2, 0, -2, -2, 4, -4]
    assert q[16:].tolist() == [1, 2, 3, -1, -2]


def test_quantize_saturates_and_maps_nan_to_zero():
    x = np.array([300.0, -300.0, 127.4, -128.6, np.inf, -np.inf, np.nan, 0.0] * 2 + [np.nan, 1e9, -1e9],
                 np.float32)
    q = quantize(x, 1.0)
    assert q[:8].tolist() == [127, -128, 127, -128, 127, -128, 0, 0]
    assert q[16:].tolist() == [0, 127, -128]


def test_quantize_scale_is_reciprocal_multiply():
    # q = round(x * (1/scale)) -- not round(x / scale); the two differ here
    scale = np.float32(0.1)
    inv = np.float32(1.0) / scale
    x = RNG.standard_normal(4096).astype(np.float32) * 5
    q = quantize(x, float(scale))
    v = (x * inv).astype(np.float32)
    n16 = x.size // 16 * 16
    want = np.clip(np.rint(v[:n16]), -128, 127).astype(np.int8)
    np.testing.assert_array_equal(q[:n16], want)


def test_int8_accumulators_match_int64_brute_force():
    N, C, H, W, M, K = 2, 7, 6, 5, 4, 3
    xq = RNG.integers(-128, 128, (N, C, H, W), dtype=np.int8)
    wq = RNG.integers(-127, 128, (M, C, K, K), dtype=np.int8)
    acc = np.zeros((N, M, 3, 3), np.int32)
    LIB.oracle_conv_int8_acc(P(xq), P(wq), P(acc), N, C, H, W, M, K, K, 3, 3, 2, 2, 1, 1, 1, 1)
    x64 = np.zeros((N, C, H + 2, W + 2), np.int64)
    x64[:, :, 1:H + 1, 1:W + 1] = xq
    want = np.zeros((N, M, 3, 3), np.int64)
    for oh in range(3):
        for ow in range(3):
            patch = x64[:, :, oh * 2:oh * 2 + K, ow * 2:ow * 2 + K]
            want[:, :, oh, ow] = np.einsum("nckl,mckl->nm", patch, wq.astype(np.int64))
    np.testing.assert_array_equal(acc, want)


def test_int8_accumulator_zero_point_identity():
    """sum w*(x - zp) == sum w*x - zp*sum w over the taps (no padding)."""
    N, C, H, W, M = 1, 5, 4, 4, 3
    xq = RNG.integers(-100, 100, (N, C, H, W), dtype=np.int8)
    wq = RNG.integers(-127, 128, (M, C, 2, 2), dtype=np.int8)
    zp = 7
    acc = np.zeros((N, M, 3, 3), np.int32)
    acc_zp = np.zeros_like(acc)
    LIB.oracle_conv_int8_acc(P(xq), P(wq), P(acc), N, C, H, W, M, 2, 2, 3, 3, 1, 1, 0, 0, 1, 1)
    xs = (xq.astype(np.int16) - zp).astype(np.int8)
    LIB.oracle_conv_int8_acc(P(xs), P(wq), P(acc_zp), N, C, H, W, M, 2, 2, 3, 3, 1, 1, 0, 0, 1, 1)
    wsum = wq.astype(np.int64).sum(axis=(1, 2, 3))
    np.testing.assert_array_equal(acc_zp, acc - zp * wsum[None, :, None, None])


def test_dequant_is_single_rounding_fma():
    """y = fmaf((float)acc, w_scale[m] * x_scale, bias[m]) -- one rounding of
    the exact acc*s + bias (conv_int8.c:86-119), checked in exact rationals."""
    M, S = 3, 40
    acc = RNG.integers(-2**20, 2**20, (1, M, S), dtype=np.int32)
    ws = RNG.uniform(0.001, 0.02, M).astype(np.float32)
    xs = np.float32(0.037)
    bias = RNG.standard_normal(M).astype(np.float32)
    y = np.zeros((1, M, S), np.float32)
    LIB.oracle_dequant(P(acc), P(ws), ctypes.c_float(xs), P(bias), None, P(y), 1, M, S, 0)
    for m in range(M):
        s = np.float32(ws[m] * xs)
        for i in range(S):
            exact = Fraction(int(acc[0, m, i])) * Fraction(float(s)) + Fraction(float(bias[m]))
            yv = y[0, m, i]
            err = abs(Fraction(float(yv)) - exact)
            for nb in (np.nextafter(yv, np.float32(np.inf)), np.nextafter(yv, np.float32(-np.inf))):
                assert err <= abs(Fraction(float(nb)) - exact), (m, i)


def test_int8_conv_end_to_end_relu_and_residual():
    N, C, H, W, M = 1, 4, 5, 5, 3
    x = RNG.standard_normal((N, C, H, W)).astype(np.float32)
    wq = RNG.integers(-127, 128, (M, C, 3, 3), dtype=np.int8)
    ws = np.full(M, 0.01, np.float32)
    xs = 0.05
    b = RNG.standard_normal(M).astype(np.float32)
    r = RNG.standard_normal((N, M, H, W)).astype(np.float32)
    y = np.zeros((N, M, H, W), np.float32)
    acc = np.zeros((N, M, H, W), np.int32)
    rc = LIB.oracle_conv2d_int8(P(x), P(wq), P(ws), ctypes.c_float(xs), P(b), P(r), P(y), P(acc), N, C, H, W, M, 3, 3,
                                H, W, 1, 1, 1, 1, 1, 1, 1)
    assert rc == 0
    q = quantize(np.ascontiguousarray(x.ravel()), xs).reshape(x.shape)
    acc2 = np.zeros_like(acc)
    LIB.oracle_conv_int8_acc(P(q), P(wq), P(acc2), N, C, H, W, M, 3, 3, H, W, 1, 1, 1, 1, 1, 1)
    np.testing.assert_array_equal(acc, acc2)
    deq = np.zeros_like(y)
    LIB.oracle_dequant(P(acc), P(ws), ctypes.c_float(xs), P(b), P(r), P(deq), N, M, H * W, 1)
    np.testing.assert_array_equal(y, deq)
    assert (y >= 0).all() and (y == 0).any()
