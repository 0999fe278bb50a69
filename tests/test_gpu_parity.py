"""GPU parity: the MI355X runtime against the CPU oracle on the same packages.

fp32 tolerance: tensor-normalized max error <= 1e-4 (FP32_TOL); selection /
copy ops (MaxPool, Add, Resize, Relu) bit-exact; INT8 accumulators and
dequantized outputs bit-exact.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest

from spinnv2_amd.spk import models, write_spk
from spinnv2_amd.spk.quantize import calibrate_activation_scales, quantize_conv_weights

from .helpers import FP32_TOL, rng_inputs, run_gpu, run_oracle, tnorm_err

pytestmark = pytest.mark.gpu

# (N, Cin, H, W, Cout, k, stride, pad, dilation, group, act, bias, residual)
CONV_CASES = [
    (1, 3, 17, 19, 8, 3, 1, 1, 1, 1, "Relu", True, False),
    (2, 16, 12, 12, 32, 1, 1, 0, 1, 1, None, True, False),
    (1, 3, 32, 32, 64, 7, 2, 3, 1, 1, "Relu", True, False),      # stem-like
    (2, 64, 14, 14, 64, 3, 1, 1, 1, 1, "Relu", True, True),      # residual + relu
    (1, 32, 15, 15, 48, 3, 2, 1, 1, 1, "Silu", True, False),
    (1, 8, 16, 16, 8, 3, 1, 2, 2, 1, None, False, False),        # dilation, no bias
    (1, 16, 10, 10, 16, 3, 1, 1, 1, 16, "Relu", True, False),    # depthwise -> direct kernel
    (1, 16, 10, 10, 32, 3, 1, 1, 1, 4, None, True, False),       # grouped
    (1, 130, 9, 9, 70, 1, 1, 0, 1, 1, "Relu", True, False),      # ragged M, K, N
    (3, 5, 7, 7, 3, 3, 1, 1, 1, 1, None, True, True),            # tiny
]


@pytest.mark.parametrize("case", CONV_CASES, ids=[f"conv{i}" for i in range(len(CONV_CASES))])
def test_conv_f32_vs_oracle(gpu, case):
    n, cin, h, w, cout, k, s, p, d, grp, act, bias, res = case
    g = models.single_conv(n, cin, h, w, cout, k, s, p, d, grp, act, bias, res)
    blob = write_spk(g, "mi355x")
    xs = rng_inputs(g)
    print(f"conv case {case}", flush=True)
    got = run_gpu(blob, xs)[0]
    want = run_oracle(blob, xs)[0]
    assert tnorm_err(got, want) <= FP32_TOL


# Depthwise convs (one input channel per group) run conv_dw_f32, which sums
# each output in the reference's order with one fused multiply-add per
# in-bounds tap, as the oracle does: bit-exact without SiLU.
# (N, C, H, W, multiplier, k, stride, pads [t, l, b, r], dilation, act, residual)
DW_CASES = [
    (1, 16, 10, 10, 1, 3, 1, [1, 1, 1, 1], 1, "Relu", False),
    (2, 32, 50, 70, 1, 3, 1, [1, 1, 1, 1], 1, None, True),     # several 16x16 tiles, residual
    (1, 24, 33, 31, 2, 5, 2, [2, 2, 2, 2], 1, "Relu", False),  # channel multiplier 2, stride 2
    (1, 8, 29, 23, 1, 7, 1, [3, 3, 3, 3], 1, None, False),      # 7x7
    (1, 8, 20, 20, 1, 3, 1, [2, 2, 2, 2], 2, "Relu", False),    # dilation 2
    (1, 8, 17, 19, 1, 3, 2, [0, 1, 1, 0], 1, None, False),      # asymmetric padding
    (16, 128, 20, 20, 1, 3, 1, [1, 1, 1, 1], 1, None, False),   # the YOLO PSA position encoding
]


@pytest.mark.parametrize("case", DW_CASES, ids=[f"dw{i}" for i in range(len(DW_CASES))])
def test_depthwise_conv_bitwise(gpu, case):
    from spinnv2_amd.runtime import Model

    n, c, h, w, mult, k, s, pads, d, act, res = case
    g = models.single_conv(n, c, h, w, c * mult, k, s, dilation=d, group=c, act=act, residual=res, pads=pads)
    blob = write_spk(g, "mi355x")
    xs = rng_inputs(g)
    with Model(blob) as m:
        for i, x in enumerate(xs):
            m.set_input(i, x)
        m.run()
        got = m.get_output(0)
        assert m.kernel_name(0) == "conv_dw_f32", m.kernel_name(0)
    want = run_oracle(blob, xs)[0]
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))


# ResNet-101 layers at their real shapes, batch 1 (split-K path) and batch 8
RESNET_LAYERS = [
    (64, 56, 64, 3, 1, 1),     # s1 3x3
    (256, 56, 64, 1, 1, 0),    # s1 1x1 reduce
    (128, 28, 128, 3, 1, 1),   # s2 3x3
    (256, 14, 256, 3, 1, 1),   # s3 3x3
    (1024, 14, 256, 1, 1, 0),  # s3 1x1 reduce
    (256, 14, 1024, 1, 1, 0),  # s3 1x1 expand
    (512, 7, 512, 3, 1, 1),    # s4 3x3
    (512, 7, 2048, 1, 1, 0),   # s4 1x1 expand
    (512, 28, 1024, 1, 2, 0),  # s3 projection 1x1/2
]


@pytest.mark.parametrize("batch", [1, 4])
@pytest.mark.parametrize("layer", RESNET_LAYERS, ids=[f"L{i}" for i in range(len(RESNET_LAYERS))])
def test_resnet_layer_shapes(gpu, layer, batch):
    cin, hw, cout, k, s, p = layer
    g = models.single_conv(batch, cin, hw, hw, cout, k, s, p, act="Relu", residual=False)
    blob = write_spk(g, "mi355x")
    xs = rng_inputs(g)
    print(f"resnet layer {layer} b={batch}", flush=True)
    got = run_gpu(blob, xs)[0]
    want = run_oracle(blob, xs)[0]
    assert tnorm_err(got, want) <= FP32_TOL


@pytest.mark.parametrize("rows,k,nout,trans_b,alpha", [(1, 400, 120, 0, 1.0), (64, 2048, 1000, 0, 1.0),
                                                       (3, 84, 10, 1, 0.5), (1, 2048, 1000, 1, 1.0)])
def test_gemm_vs_oracle(gpu, rows, k, nout, trans_b, alpha):
    g = models.single_gemm(rows, k, nout, alpha=alpha, trans_b=trans_b)
    blob = write_spk(g, "mi355x")
    xs = rng_inputs(g)
    got = run_gpu(blob, xs)[0]
    want = run_oracle(blob, xs)[0]
    assert tnorm_err(got, want) <= FP32_TOL


EXACT_OPS = [
    ("MaxPool", [2, 8, 23, 23], dict(k=3, s=2, p=1)),
    ("MaxPool", [1, 4, 8, 8], dict(k=2, s=2, p=0)),
    ("Add", [2, 16, 9, 9], {}),
    ("Add", [2, 16, 9, 9], dict(b_shape=[1, 16, 1, 1])),
    ("Add", [1, 8, 5, 5], dict(relu=True)),
    ("Relu", [3, 7, 11], {}),
    ("Resize", [1, 4, 10, 12], dict(scale=2)),
    # the vectorized 3x3/s2/p1 MaxPool (W % 8 == 0) and 2x Resize (W even) paths, and an odd-W Resize
    ("MaxPool", [2, 8, 32, 48], dict(k=3, s=2, p=1)),
    ("MaxPool", [1, 3, 16, 8], dict(k=3, s=2, p=1)),
    ("Resize", [2, 3, 6, 10], dict(scale=2)),
    ("Resize", [2, 3, 5, 7], dict(scale=2)),
    # one operand a single element (16-byte path), either order; odd size (generic path)
    ("Mul", [2, 3, 40, 40], dict(b_shape=[1])),
    ("Sub", [2, 3, 40, 40], dict(b_shape=[1], swap=True)),
    ("Div", [2, 8, 10, 10], dict(b_shape=[1], swap=True)),
    ("Mul", [3, 5, 7], dict(b_shape=[1])),
    # the unrolled-window pools: SPPF's 5x5/1/2, a 3x3/1/1 and a 5x5/2/2 on odd sizes; a 4x4 window
    # stays on the generic loop
    ("MaxPool", [2, 16, 20, 20], dict(k=5, s=1, p=2)),
    ("MaxPool", [1, 8, 13, 11], dict(k=3, s=1, p=1)),
    ("MaxPool", [1, 8, 17, 15], dict(k=5, s=2, p=2)),
    ("MaxPool", [1, 4, 12, 12], dict(k=4, s=2, p=1)),
]


@pytest.mark.parametrize("op,shape,kw", EXACT_OPS, ids=[f"{o}{i}" for i, (o, _, _) in enumerate(EXACT_OPS)])
def test_exact_ops_bitwise(gpu, op, shape, kw):
    g = models.single_op(op, shape, **kw)
    blob = write_spk(g, "mi355x")
    xs = rng_inputs(g)
    got = run_gpu(blob, xs)[0]
    want = run_oracle(blob, xs)[0]
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("k,s,p", [(2, 2, 0), (3, 1, 1), (5, 1, 2), (3, 2, 1), (4, 2, 1)])
def test_maxpool_signed_zero_order(gpu, k, s, p):
    """Windows of -0.0, +0.0 and negatives (and a NaN): the maximum of a
    window holding both zeros is whichever comes first in the reference's
    order (rows, then columns, strict >), NaN is never taken; every pooling
    kernel gives the oracle's bits."""
    g = models.single_op("MaxPool", [2, 3, 16, 16], k=k, s=s, p=p)
    blob = write_spk(g, "mi355x")
    rng = np.random.default_rng(k * 10 + s)
    x = rng.choice(np.array([-0.0, 0.0, -1.5, -0.25], np.float32), size=(2, 3, 16, 16))
    x[0, 0, 3, 5] = np.nan
    got = run_gpu(blob, [x])[0]
    want = run_oracle(blob, [x])[0]
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))


FLOAT_OPS = [
    ("Softmax", [4, 1000], dict(axis=-1)),
    ("Softmax", [2, 16, 50], dict(axis=1)),
    ("Softmax", [5, 2048], dict(axis=-1)),     # register-resident rows at their limit
    ("Softmax", [4099, 1000], dict(axis=-1)),  # many rows (non-temporal stores)
    ("Softmax", [1100, 2048], dict(axis=-1)),  # many long rows (non-temporal stores)
    ("Softmax", [2048, 36], dict(axis=-1)),    # many short rows
    ("Softmax", [3, 2052], dict(axis=-1)),     # longer rows: three passes
    ("Softmax", [3, 6, 7], dict(axis=-1)),     # rows not a multiple of 4
    ("Softmax", [2, 16, 4, 300], dict(axis=1)),  # DFL-like: 16 strided bins in registers
    ("Softmax", [2, 24, 70], dict(axis=1)),    # strided, 24 of up to 32 in registers
    ("Softmax", [2, 40, 33], dict(axis=1)),    # strided, longer than the register forms
    ("ReduceMean", [4, 2048, 7, 7], dict(axes=[2, 3])),
    ("ReduceMean", [2, 6, 5, 4], dict(axes=[1])),
    ("GlobalAveragePool", [2, 32, 7, 7], {}),
    ("AveragePool", [1, 4, 9, 9], dict(k=3, s=2, p=1)),
    ("Sigmoid", [2, 300], {}),
    ("Sigmoid", [3, 7, 5], {}),                # odd size: one element per thread
    ("Mul", [2, 8, 4, 4], dict(b_shape=[8, 1, 1])),
]


@pytest.mark.parametrize("op,shape,kw", FLOAT_OPS, ids=[f"{o}{i}" for i, (o, _, _) in enumerate(FLOAT_OPS)])
def test_float_ops(gpu, op, shape, kw):
    g = models.single_op(op, shape, **kw)
    blob = write_spk(g, "mi355x")
    xs = rng_inputs(g)
    got = run_gpu(blob, xs)[0]
    want = run_oracle(blob, xs)[0]
    assert tnorm_err(got, want) <= 1e-5


def test_lenet_e2e(gpu):
    g = models.lenet()
    blob = write_spk(g, "mi355x")
    xs = rng_inputs(g, dist="uniform")
    got = run_gpu(blob, xs)[0]
    want = run_oracle(blob, xs)[0]
    assert tnorm_err(got, want) <= FP32_TOL
    assert np.argmax(got) == np.argmax(want)


def test_resnet18_e2e_b1(gpu):
    g = models.resnet(18, 1)
    blob = write_spk(g, "mi355x")
    xs = rng_inputs(g)
    got = run_gpu(blob, xs)[0]
    want = run_oracle(blob, xs)[0]
    assert tnorm_err(got, want) <= FP32_TOL
    assert np.argmax(got) == np.argmax(want)


def test_resnet101_e2e_b1(gpu):
    """The benchmark network at batch 1 against the oracle."""
    g = models.resnet(101, 1)
    blob = write_spk(g, "mi355x")
    xs = rng_inputs(g)
    got = run_gpu(blob, xs)[0]
    want = run_oracle(blob, xs)[0]
    assert tnorm_err(got, want) <= FP32_TOL
    assert np.argmax(got) == np.argmax(want)


def test_resnet101_b64_images_match_batch1(gpu):
    """The benchmark configuration itself (ResNet-101, 224x224, batch 64):
    every image is independent through every node, so images 0 and 63 of
    the batch-64 run must agree with batch-1 runs of the same images (other
    tiles and split-K choices, so within the fp32 tolerance), and image 0
    with the oracle."""
    g64 = models.resnet(101, 64)
    x = rng_inputs(g64)[0]
    out64 = run_gpu(write_spk(g64, "mi355x"), [x])[0].reshape(64, -1)
    g1 = models.resnet(101, 1)
    blob1 = write_spk(g1, "mi355x")
    for i in (0, 63):
        one = run_gpu(blob1, [x[i:i + 1]])[0]
        assert tnorm_err(out64[i], one) <= FP32_TOL, i
        assert np.argmax(out64[i]) == np.argmax(one), i
    want0 = run_oracle(blob1, [x[0:1]])[0]
    assert tnorm_err(out64[0], want0) <= FP32_TOL
    assert np.argmax(out64[0]) == np.argmax(want0)


def test_cpu_generic_package_runs_on_gpu(gpu):
    """A package compiled for cpu_generic (bnns / simd kinds) runs unchanged."""
    g = models.resnet(18, 1)
    xs = rng_inputs(g)
    got_generic = run_gpu(write_spk(g, "cpu_generic"), xs)[0]
    got_mi = run_gpu(write_spk(g, "mi355x"), xs)[0]
    np.testing.assert_array_equal(got_generic, got_mi)


INT8_CASES = [
    dict(n=1, cin=16, h=14, w=14, cout=32, k=3, stride=1, pad=1, act="Relu"),
    dict(n=2, cin=64, h=14, w=14, cout=64, k=1, stride=1, pad=0, act=None, residual=True),
    dict(n=1, cin=3, h=32, w=32, cout=64, k=7, stride=2, pad=3, act="Relu"),      # stem: (kw, c) runs, C % 4 != 0
    dict(n=1, cin=128, h=7, w=7, cout=256, k=3, stride=2, pad=1, act="Relu"),     # small grid
    dict(n=1, cin=20, h=9, w=9, cout=24, k=3, stride=1, pad=2, dilation=2, act=None),  # per-tap groups, C padded
    dict(n=2, cin=40, h=10, w=12, cout=30, k=3, stride=1, pad=0, act="Relu", pads=[1, 0, 0, 2]),  # asymmetric pads
    dict(n=3, cin=256, h=7, w=7, cout=512, k=1, stride=1, pad=0, act="Relu", residual=True),
]


def _int8_check(g, seed=42):
    from spinnv2_amd.runtime import Model
    from oracle.spk_exec import OracleExecutor

    xs = rng_inputs(g, seed)
    qp = calibrate_activation_scales(g, [xs]) + quantize_conv_weights(g)
    blob = write_spk(g, "mi355x", quant_params=qp)
    ora = OracleExecutor(blob)
    want = ora.run(*xs)[0].ravel()
    with Model(blob) as m:
        for i, x in enumerate(xs):
            m.set_input(i, x)
        m.run()
        got = m.get_output(0)
        acc = m.int8_accumulators(0, want.nbytes)
        name = m.kernel_name(0)
    np.testing.assert_array_equal(acc, ora.acc[0].ravel())
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))
    return name


@pytest.mark.parametrize("case", INT8_CASES, ids=[f"i8_{i}" for i in range(len(INT8_CASES))])
def test_int8_conv_bit_exact(gpu, case):
    print(f"[int8] {case}", flush=True)
    _int8_check(models.single_conv(**case))


I8_FORCED = [(cfg, split) for cfg in range(7) for split in (1, 3)]


@pytest.mark.parametrize("cfg,split", I8_FORCED, ids=[f"i8cfg{c}_split{s}" for c, s in I8_FORCED])
def test_int8_every_tile_config_and_split(gpu, monkeypatch, cfg, split):
    monkeypatch.setenv("SPKV2_I8_CFG", str(cfg))
    monkeypatch.setenv("SPKV2_I8_SPLITK", str(split))
    name = _int8_check(models.single_conv(2, 48, 11, 13, 70, 3, 1, 1, act="Relu", residual=True))
    # the effective split is capped by the layer's k-tile count
    assert ("splitk=1>" in name) == (split == 1), name


# Pixel-major gather configurations (7-13, the direct-weight kernel
# conv_igemm_i8x: 14-22 and 31-34, and its persistent form conv_igemm_i8p:
# 23-30 and 35-36, which takes whole tiles only): every one on a 1x1 conv
# (one kernel row: always eligible) and on a 3x3 conv with 64 channels (12
# groups per kernel row: eligible for BK = 64 only), with split-K, ragged M
# and N, residual and Relu; ineligible forcings are refused.
I8_PX_BK = {7: 64, 8: 128, 9: 64, 10: 128, 11: 64, 12: 64, 13: 128,
            14: 128, 15: 128, 16: 128, 17: 128, 18: 64, 19: 64, 20: 64, 21: 64, 22: 128,
            23: 64, 24: 64, 25: 64, 26: 64, 27: 128, 28: 128, 29: 64, 30: 128,
            31: 64, 32: 128, 33: 64, 34: 128, 35: 64, 36: 128}
I8_PERSIST = {*range(23, 31), 35, 36}
I8_PX = [(cfg, shape, split) for cfg in I8_PX_BK for shape in ("1x1", "3x3") for split in (1, 3)]


@pytest.mark.parametrize("cfg,shape,split", I8_PX, ids=[f"i8px{c}_{s}_split{k}" for c, s, k in I8_PX])
def test_int8_pixel_gather_configs(gpu, monkeypatch, cfg, shape, split):
    from spinnv2_amd.runtime import RuntimeError_

    monkeypatch.setenv("SPKV2_I8_CFG", str(cfg))
    monkeypatch.setenv("SPKV2_I8_SPLITK", str(split))
    if shape == "1x1":
        g = models.single_conv(3, 96, 9, 11, 70, 1, 1, 0, act="Relu", residual=True)
    else:
        g = models.single_conv(2, 64, 11, 13, 70, 3, 1, 1, act="Relu", residual=True)
    if shape == "3x3" and I8_PX_BK[cfg] == 128:
        with pytest.raises(RuntimeError_) as e:
            _int8_check(g)
        assert e.value.code == -32
        return
    name = _int8_check(g)
    assert (",ax" in name) if cfg >= 14 else (",px," in name), name
    assert (",persist" in name) == (cfg in I8_PERSIST), name


def test_graph_mode_matches_eager(gpu):
    from spinnv2_amd.runtime import Model

    g = models.resnet(18, 2)
    blob = write_spk(g, "mi355x")
    xs = rng_inputs(g)
    with Model(blob) as m:
        m.set_input(0, xs[0])
        m.run()
        eager = m.get_output(0)
        m.set_graph_mode(True)
        for _ in range(3):
            m.set_input(0, xs[0])
            m.run()
            np.testing.assert_array_equal(m.get_output(0), eager)


# Every implicit-GEMM tile configuration (the fp32 table of conv_f32.hip: 8
# shallow-k tiles, 4 deep-k ones, then after the two skinny kernels 3 tiles
# of 32 rows, after the two thin ones 2 tiles of 96 rows, and after the
# row-window and sixteen-wave entries 2 tiles with the waves along M), with
# and without split-K (each slice writes its partial tile; splitk_epilogue
# sums them in slice order and applies the epilogue), on a ragged residual
# conv; forced through the tuning overrides.
F32_IGEMM_CFGS = [*range(12), 14, 15, 16, 19, 20, 25, 26]
F32_SKINNY_CFGS = [12, 13, 23]  # 4, 8 and 16 waves
SKINNY_WAVES = {12: 4, 13: 8, 23: 16}
SPLIT_CASES = [(cfg, split) for cfg in F32_IGEMM_CFGS for split in (1, 3, 8)]


@pytest.mark.parametrize("cfg,split", SPLIT_CASES, ids=[f"cfg{c}_split{s}" for c, s in SPLIT_CASES])
def test_conv_every_tile_config_and_split(gpu, monkeypatch, cfg, split):
    monkeypatch.setenv("SPKV2_CONV_CFG", str(cfg))
    monkeypatch.setenv("SPKV2_CONV_SPLITK", str(split))
    g = models.single_conv(2, 72, 11, 13, 150, 3, 1, 1, act="Relu", residual=True)
    blob = write_spk(g, "mi355x")
    xs = rng_inputs(g)
    got = run_gpu(blob, xs)[0]
    want = run_oracle(blob, xs)[0]
    assert tnorm_err(got, want) <= FP32_TOL


# Padded convs whose input no producer hands over padded: implicit padding
# (every tap bounds-checked against the unpadded input; forced here with
# SPKV2_IMPLICIT_PAD=1, by default only for short gathers) or, with
# SPKV2_IMPLICIT_PAD=0, a zero-padded copy first.
# (N, Cin, H, W, Cout, k, stride, pads [t, l, b, r], dilation, residual)
PAD_CASES = [
    (2, 16, 13, 11, 40, 3, 1, [1, 1, 1, 1], 1, True),
    (1, 3, 37, 29, 16, 3, 2, [1, 1, 1, 1], 1, False),   # YOLO-stem-like: 3 channels, stride 2
    (1, 3, 30, 30, 64, 7, 2, [3, 3, 3, 3], 1, False),   # ResNet-stem-like
    (1, 8, 17, 19, 24, 3, 1, [0, 2, 1, 0], 1, False),   # asymmetric
    (1, 8, 20, 20, 24, 3, 1, [2, 2, 2, 2], 2, True),    # dilation 2
]


@pytest.mark.parametrize("implicit", ["1", "0"])
@pytest.mark.parametrize("cfg", [6, 7, 8, 14])
@pytest.mark.parametrize("case", PAD_CASES, ids=[f"pad{i}" for i in range(len(PAD_CASES))])
def test_padded_conv_implicit_and_copied(gpu, monkeypatch, case, cfg, implicit):
    from spinnv2_amd.runtime import Model

    monkeypatch.setenv("SPKV2_CONV_CFG", str(cfg))
    monkeypatch.setenv("SPKV2_IMPLICIT_PAD", implicit)
    monkeypatch.setenv("SPKV2_CONV_SMALLK", "0")  # the 3-channel stem shapes on the implicit GEMM
    n, c, h, w, m, k, s, pads, d, res = case
    g = models.single_conv(n, c, h, w, m, k, s, dilation=d, act="Relu", residual=res, pads=pads)
    blob = write_spk(g, "mi355x")
    xs = rng_inputs(g)
    with Model(blob) as mdl:
        for i, x in enumerate(xs):
            mdl.set_input(i, x)
        mdl.run()
        got = mdl.get_output(0)
        name = mdl.kernel_name(0)
    if implicit == "1":
        assert ",ipad" in name, name
    else:
        assert ",pad" in name and ",ipad" not in name, name
    assert tnorm_err(got, run_oracle(blob, xs)[0]) <= FP32_TOL


@pytest.mark.parametrize("smallk", ["1", "0"])
def test_silu_activation_accuracy(gpu, monkeypatch, smallk):
    """The fused SiLU (hardware exponential and reciprocal) against
    v / (1 + exp(-v)) in float64: a 1x1 conv with weight 1 and bias 0 passes
    every input through unchanged, then the activation; within 1e-5 relative
    (0.5e-5 absolute near 0) on a grid over [-100, 100], and the special
    values exactly (+inf, -inf -> NaN, NaN, -0 below about -88.7).  Both the
    small-gather kernel and the implicit GEMM's epilogue."""
    from spinnv2_amd.spk.graph import Graph
    from spinnv2_amd.spk.passes import run_default_pipeline

    monkeypatch.setenv("SPKV2_CONV_SMALLK", smallk)
    grid = np.concatenate([np.linspace(-100, 100, 20001), [-88.5, -89.0, -90.0, 0.0, -0.0, 1e-30, -1e-30, 87.0, 89.0]])
    specials = np.array([np.inf, -np.inf, np.nan])
    x = np.concatenate([grid, specials, np.zeros(128 - (grid.size + 3) % 128)]).astype(np.float32)
    g = Graph("silu")
    xi = g.input("x", [1, 1, x.size // 128, 128])
    g.mark_output(g.silu(g.conv(xi, np.ones((1, 1, 1, 1), np.float32), np.zeros(1, np.float32))))
    run_default_pipeline(g)
    got = run_gpu(write_spk(g, "mi355x"), [x.reshape(1, 1, -1, 128)])[0].ravel()
    xd = x.astype(np.float64)
    with np.errstate(over="ignore", invalid="ignore"):
        want = xd / (1.0 + np.exp(-xd))
    fin = np.isfinite(xd)
    np.testing.assert_allclose(got[fin], want[fin], rtol=1e-5, atol=0.5e-5)
    assert got[grid.size] == np.inf and np.isnan(got[grid.size + 1]) and np.isnan(got[grid.size + 2])
    assert np.all(got[:grid.size][x[:grid.size] < -89.0] == 0.0)


# Batched MatMul through both kernels: 64x64 LDS tiles and 32x32 tiles with
# k split over the waves (chosen when the 64x64 grid is small; forced here):
# plain 2-D, batched, broadcasting both ways, a constant B, ragged tiles,
# K not a multiple of 8 or of 32, and the PSA attention products.
MATMUL_CASES = [
    dict(a_shape=[5, 7], b_shape=[7, 3]),
    dict(a_shape=[2, 3, 8, 16], b_shape=[2, 3, 16, 5]),
    dict(a_shape=[2, 1, 4, 6], b_shape=[3, 6, 5]),
    dict(a_shape=[3, 70, 33], b_shape=[33, 65]),
    dict(a_shape=[4, 33, 17], b_shape=[17, 9], const_b=True),
    dict(a_shape=[1, 2, 400, 32], b_shape=[1, 2, 32, 400]),
    dict(a_shape=[1, 2, 64, 400], b_shape=[1, 2, 400, 400]),
    dict(a_shape=[2, 40, 1001], b_shape=[1001, 37]),
]


@pytest.mark.parametrize("ksplit", ["1", "0"])
@pytest.mark.parametrize("kw", MATMUL_CASES, ids=[f"mm{i}" for i in range(len(MATMUL_CASES))])
def test_matmul_both_kernels(gpu, monkeypatch, kw, ksplit):
    from spinnv2_amd.runtime import Model

    monkeypatch.setenv("SPKV2_MATMUL_KSPLIT", ksplit)
    g = models.matmul_op(**kw)
    blob = write_spk(g, "mi355x")
    xs = rng_inputs(g)
    with Model(blob) as m:
        for i, x in enumerate(xs):
            m.set_input(i, x)
        m.run()
        got = m.get_output(0)
        name = m.kernel_name(0)
    assert ("ksplit" in name) == (ksplit == "1"), name
    assert tnorm_err(got, run_oracle(blob, xs)[0]) <= FP32_TOL


def test_sigmoid_accuracy(gpu):
    """Sigmoid (hardware exponential and reciprocal, 16-byte path) against
    1 / (1 + exp(-v)) in float64: within 1e-5 relative on a grid over
    [-100, 100]; +inf -> 1, -inf -> 0, NaN -> NaN."""
    grid = np.linspace(-100, 100, 20001)
    x = np.concatenate([grid, [np.inf, -np.inf, np.nan], np.zeros(1)]).astype(np.float32)
    g = models.single_op("Sigmoid", [1, x.size])
    got = run_gpu(write_spk(g, "mi355x"), [x.reshape(1, -1)])[0].ravel()
    want = 1.0 / (1.0 + np.exp(-grid))
    np.testing.assert_allclose(got[:grid.size], want, rtol=1e-5, atol=1e-30)
    assert got[grid.size] == 1.0 and got[grid.size + 1] == 0.0 and np.isnan(got[grid.size + 2])


# Small-gather stems (conv_smallk_f32: at most 4 input channels and 64 taps,
# at most 64 output channels; one output pixel per lane, every output channel
# in registers), against the oracle and against the implicit GEMM.
# (N, Cin, H, W, Cout, k, stride, pads [t, l, b, r], dilation, residual, act)
SMALLK_CASES = [
    (2, 3, 37, 29, 16, 3, 2, [1, 1, 1, 1], 1, False, "Silu"),  # YOLO stem
    (1, 1, 28, 28, 6, 5, 1, [0, 0, 0, 0], 1, False, "Relu"),   # LeNet conv1
    (3, 4, 20, 70, 40, 4, 1, [2, 1, 1, 2], 1, True, "Relu"),   # 64 taps, asymmetric pads, residual
    (1, 2, 33, 130, 64, 3, 1, [2, 2, 2, 2], 2, False, None),   # dilation 2, rows of 3 segments
    (2, 3, 9, 9, 24, 3, 3, [0, 0, 0, 0], 1, True, "Relu"),     # stride 3, short rows
]


@pytest.mark.parametrize("case", SMALLK_CASES, ids=[f"smallk{i}" for i in range(len(SMALLK_CASES))])
def test_smallk_stem_conv(gpu, monkeypatch, case):
    from spinnv2_amd.runtime import Model

    n, c, h, w, m, k, s, pads, d, res, act = case
    g = models.single_conv(n, c, h, w, m, k, s, dilation=d, act=act, residual=res, pads=pads)
    blob = write_spk(g, "mi355x")
    xs = rng_inputs(g)
    print(f"[smallk] case {case}", flush=True)
    outs = {}
    for flag in ("1", "0"):
        monkeypatch.setenv("SPKV2_CONV_SMALLK", flag)
        with Model(blob) as mdl:
            for i, x in enumerate(xs):
                mdl.set_input(i, x)
            mdl.run()
            outs[flag] = mdl.get_output(0)
            name = mdl.kernel_name(0)
        assert (name == "conv_smallk_f32") == (flag == "1"), name
    want = run_oracle(blob, xs)[0]
    assert tnorm_err(outs["1"], want) <= FP32_TOL
    assert tnorm_err(outs["1"], outs["0"]) <= FP32_TOL


def test_smallk_stem_handoff_graph_mode(gpu, monkeypatch):
    """A stem on the small-gather kernel hands its output to the padded 3x3
    conv after it (stored straight into that conv's zero-padded input, the
    tensor itself not written when nothing else reads it); eager, HIP-graph
    replays and the handoff switched off agree bit for bit."""
    from spinnv2_amd.runtime import Model
    from spinnv2_amd.spk.graph import Graph
    from spinnv2_amd.spk.passes import run_default_pipeline

    p = models.Params(9)
    g = Graph("stem_handoff")
    x = g.input("x", [2, 3, 48, 40])
    a = g.silu(g.conv(x, p.he((16, 3, 3, 3)), p.normal(16, 0.01), stride=2, pad=1))
    b = g.silu(g.conv(a, p.he((32, 16, 3, 3)), p.normal(32, 0.01), stride=2, pad=1))
    g.mark_output(b)
    run_default_pipeline(g)
    blob = write_spk(g, "mi355x")
    xs = rng_inputs(g)
    outs = {}
    for flag in ("1", "0"):
        monkeypatch.setenv("SPKV2_PAD_HANDOFF", flag)
        with Model(blob) as m:
            m.set_input(0, xs[0])
            m.run()
            eager = m.get_output(0)
            names = [m.kernel_name(nd.id) for nd in g.nodes if nd.op_type == "Conv"]
            m.set_graph_mode(True)
            for _ in range(3):
                m.set_input(0, xs[0])
                m.run()
                np.testing.assert_array_equal(m.get_output(0), eager)
        outs[flag] = eager
        assert names[0] == "conv_smallk_f32", names
        assert names[1].endswith("+handoff") == (flag == "1"), names
    np.testing.assert_array_equal(outs["1"], outs["0"])
    assert tnorm_err(outs["1"], run_oracle(blob, xs)[0]) <= FP32_TOL


@pytest.mark.parametrize("cfg", F32_IGEMM_CFGS)
@pytest.mark.parametrize("k", [136, 130])
def test_gemm_every_tile_config(gpu, monkeypatch, cfg, k):
    """Gemm through every implicit-GEMM tile: with K a multiple of 4 the B
    operand (A, [rows][K]) is loaded 16 bytes along k at a time (the KVEC
    instances), otherwise one element at a time; ragged M and N."""
    monkeypatch.setenv("SPKV2_CONV_CFG", str(cfg))
    g = models.single_gemm(70, k, 90, alpha=0.75)
    blob = write_spk(g, "mi355x")
    xs = rng_inputs(g)
    assert tnorm_err(run_gpu(blob, xs)[0], run_oracle(blob, xs)[0]) <= FP32_TOL


# The skinny configurations (16 x 16 tiles, k over 4, 8 or 16 waves summed
# in LDS; entries 12, 13 and 23 of the fp32 table) on layers whose channels per tap
# are multiples of 64: ragged M and N, padding, stride, dilation, residual,
# and Gemm with alpha and with transA.
SKINNY_CASES = [
    ("conv3x3_res", lambda: models.single_conv(2, 128, 11, 13, 150, 3, 1, 1, act="Relu", residual=True)),
    ("conv1x1_s2", lambda: models.single_conv(1, 256, 14, 14, 72, 1, 2, 0, act=None)),
    # 6 chunks of 64 k: with 4 waves two chunks in flight per wave and two
    # waves multiplying one chunk of zeros; with 8 waves two waves idle
    ("conv1x1_c384", lambda: models.single_conv(1, 384, 9, 10, 50, 1, 1, 0, act="Relu")),
    ("conv3x3_s2_dil2", lambda: models.single_conv(1, 64, 15, 15, 40, 3, 2, 2, dilation=2, act="Relu")),
    ("gemm_alpha", lambda: models.single_gemm(3, 192, 70, alpha=0.5)),
    ("gemm_trans_a", lambda: models.single_gemm(5, 128, 33, trans_a=1)),
]


@pytest.mark.parametrize("cfg", F32_SKINNY_CFGS)
@pytest.mark.parametrize("name,build", SKINNY_CASES, ids=[c[0] for c in SKINNY_CASES])
def test_skinny_configs(gpu, monkeypatch, cfg, name, build):
    from spinnv2_amd.runtime import Model

    monkeypatch.setenv("SPKV2_CONV_CFG", str(cfg))
    g = build()
    blob = write_spk(g, "mi355x")
    xs = rng_inputs(g)
    with Model(blob) as m:
        for i, x in enumerate(xs):
            m.set_input(i, x)
        m.run()
        got = m.get_output(0)
        name = m.kernel_name(0)
    assert f"conv_skinny_f32<16x16,w{SKINNY_WAVES[cfg]}," in name or f"conv_skinny_f32<16x16,w{SKINNY_WAVES[cfg]}>" in name, name
    want = run_oracle(blob, xs)[0]
    assert tnorm_err(got, want) <= FP32_TOL


# The row-window configurations (entries 21, 22 and 24: the skinny kernels'
# arithmetic with 4, 8 and 16 waves, one output row segment per workgroup,
# the input window in LDS)
# on convolutions: several images and rows, rows narrower and wider than a
# 16-pixel segment (a partial last segment), stride 2, dilation, residual, a
# 1x1 layer whose waves hold unequal chunk counts, and a 512-channel window.
F32_WINDOW_CFGS = [21, 22, 24]
WINDOW_CASES = [
    ("conv3x3_res", lambda: models.single_conv(2, 128, 11, 13, 150, 3, 1, 1, act="Relu", residual=True)),
    ("conv3x3_s2", lambda: models.single_conv(1, 128, 29, 29, 40, 3, 2, 1, act="Relu")),
    ("conv3x3_dil2_wide", lambda: models.single_conv(1, 64, 20, 40, 24, 3, 1, 2, dilation=2, act=None)),
    ("conv1x1_c384", lambda: models.single_conv(1, 384, 9, 10, 50, 1, 1, 0, act="Relu")),
    ("conv1x1_s2", lambda: models.single_conv(1, 256, 14, 14, 72, 1, 2, 0, act=None)),
    ("conv3x3_c512_res", lambda: models.single_conv(1, 512, 7, 7, 64, 3, 1, 1, act="Relu", residual=True)),
    # windows narrow enough that whole waves load no window channel (16
    # waves x 8 rows, and 8 waves x 16 rows, against 64 channels): those
    # waves still load their weights
    ("conv3x3_c64_5x5", lambda: models.single_conv(2, 64, 5, 5, 64, 3, 1, 1, act="Relu")),
    ("conv1x1_c64_4x4", lambda: models.single_conv(1, 64, 4, 4, 32, 1, 1, 0, act=None)),
]


def _run_named(blob, xs):
    from spinnv2_amd.runtime import Model

    with Model(blob) as m:
        for i, x in enumerate(xs):
            m.set_input(i, x)
        m.run()
        return m.get_output(0), m.kernel_name(0)


@pytest.mark.parametrize("wi", [0, 1, 2], ids=["w4", "w8", "w16"])
@pytest.mark.parametrize("name,build", WINDOW_CASES, ids=[c[0] for c in WINDOW_CASES])
def test_window_configs_match_skinny_bit_for_bit(gpu, monkeypatch, wi, name, build):
    """Against the oracle within the fp32 tolerance, and bit for bit against
    the skinny kernel of the same wave count: both sum the same products in
    the same order (64-k chunks round robin over the waves, 16 MFMAs per
    chunk, the wave partials in wave order)."""
    g = build()
    blob = write_spk(g, "mi355x")
    xs = rng_inputs(g)
    monkeypatch.setenv("SPKV2_CONV_CFG", str(F32_WINDOW_CFGS[wi]))
    got, kname = _run_named(blob, xs)
    waves = SKINNY_WAVES[F32_SKINNY_CFGS[wi]]
    assert f"conv_window_f32<16x16,w{waves}," in kname or f"conv_window_f32<16x16,w{waves}>" in kname, kname
    assert tnorm_err(got, run_oracle(blob, xs)[0]) <= FP32_TOL
    monkeypatch.setenv("SPKV2_CONV_CFG", str(F32_SKINNY_CFGS[wi]))
    ref, kname = _run_named(blob, xs)
    assert f"conv_skinny_f32<16x16,w{waves}," in kname or f"conv_skinny_f32<16x16,w{waves}>" in kname, kname
    np.testing.assert_array_equal(got, ref)


def test_window_config_refused_where_it_does_not_fit(gpu, monkeypatch):
    """A window larger than the kernel's LDS (1024 channels x 3 rows x 19
    columns) and a Gemm (no rows) do not take a forced row-window
    configuration; both still match the oracle."""
    monkeypatch.setenv("SPKV2_CONV_CFG", str(F32_WINDOW_CFGS[0]))
    for g in (models.single_conv(1, 1024, 16, 16, 32, 3, 1, 1), models.single_gemm(3, 192, 70, alpha=0.5)):
        blob = write_spk(g, "mi355x")
        xs = rng_inputs(g)
        got, kname = _run_named(blob, xs)
        assert "window" not in kname, kname
        assert tnorm_err(got, run_oracle(blob, xs)[0]) <= FP32_TOL


@pytest.mark.parametrize("rows,k,n", [(1, 2048, 1000), (2, 132, 37), (3, 516, 70), (4, 64, 1)])
def test_gemm_matrix_vector_kernel(gpu, rows, k, n):
    """A Gemm of 1-4 rows (a classifier at batch 1-4) runs as a matrix-vector
    product (one wave per output, 16-byte weight pieces): the oracle within
    the fp32 tolerance, with alpha and bias, ragged K and outputs."""
    g = models.single_gemm(rows, k, n, alpha=0.75)
    blob = write_spk(g, "mi355x")
    xs = rng_inputs(g)
    got, kname = _run_named(blob, xs)
    assert f"gemv_f32<{rows}>" in kname, kname
    assert tnorm_err(got, run_oracle(blob, xs)[0]) <= FP32_TOL


@pytest.mark.parametrize("rows,k,trans_a", [(2, 130, 0), (3, 128, 1), (5, 128, 0)], ids=["k130", "trans_a", "rows5"])
def test_gemm_matrix_vector_kernel_not_taken(gpu, rows, k, trans_a):
    """K not a multiple of 4, a transposed A and five rows keep the tiles."""
    g = models.single_gemm(rows, k, 20, trans_a=trans_a)
    blob = write_spk(g, "mi355x")
    xs = rng_inputs(g)
    got, kname = _run_named(blob, xs)
    assert "gemv" not in kname, kname
    assert tnorm_err(got, run_oracle(blob, xs)[0]) <= FP32_TOL


def test_skinny_config_refused_off_64_channel_layers(gpu, monkeypatch):
    """A layer whose channels per tap are not a multiple of 64 does not take
    a forced skinny configuration (its chunks would straddle taps)."""
    from spinnv2_amd.runtime import Model

    monkeypatch.setenv("SPKV2_CONV_CFG", str(F32_SKINNY_CFGS[0]))
    g = models.single_conv(1, 72, 11, 13, 40, 3, 1, 1)
    blob = write_spk(g, "mi355x")
    xs = rng_inputs(g)
    with Model(blob) as m:
        m.set_input(0, xs[0])
        m.run()
        got = m.get_output(0)
        assert "skinny" not in m.kernel_name(0)
    assert tnorm_err(got, run_oracle(blob, xs)[0]) <= FP32_TOL


# The thin kernel (entries 17 and 18 of the fp32 table: 16 or 32 rows by
# 256 columns, one wave per 64 columns, no LDS) on layers whose channels per
# tap are multiples of 4: ragged M and N, padding, stride, dilation,
# residual, SiLU, and Gemm with alpha and with transA.
F32_THIN_CFGS = [17, 18]
THIN_CASES = [
    ("conv3x3_res", lambda: models.single_conv(2, 72, 11, 13, 40, 3, 1, 1, act="Relu", residual=True)),
    ("conv1x1_s2", lambda: models.single_conv(1, 32, 14, 14, 24, 1, 2, 0, act=None)),
    ("conv3x3_s2_dil2", lambda: models.single_conv(1, 16, 15, 15, 16, 3, 2, 2, dilation=2, act="Relu")),
    ("conv3x3_silu_wide", lambda: models.single_conv(2, 16, 40, 36, 32, 3, 1, 1, act="Silu")),
    ("conv5x5_c8", lambda: models.single_conv(3, 8, 17, 19, 20, 5, 1, 2, act="Relu")),
    ("gemm_alpha", lambda: models.single_gemm(3, 192, 70, alpha=0.5)),
    ("gemm_trans_a", lambda: models.single_gemm(5, 128, 33, trans_a=1)),
]


@pytest.mark.parametrize("cfg", F32_THIN_CFGS)
@pytest.mark.parametrize("name,build", THIN_CASES, ids=[c[0] for c in THIN_CASES])
def test_thin_configs(gpu, monkeypatch, cfg, name, build):
    from spinnv2_amd.runtime import Model

    monkeypatch.setenv("SPKV2_CONV_CFG", str(cfg))
    g = build()
    blob = write_spk(g, "mi355x")
    xs = rng_inputs(g)
    print(f"[thin] cfg {cfg} case {name}", flush=True)
    with Model(blob) as m:
        for i, x in enumerate(xs):
            m.set_input(i, x)
        m.run()
        got = m.get_output(0)
        kname = m.kernel_name(0)
    assert f"conv_thin_f32<thin{16 if cfg == F32_THIN_CFGS[0] else 32}x256" in kname, kname
    want = run_oracle(blob, xs)[0]
    assert tnorm_err(got, want) <= FP32_TOL


def test_thin_config_refused_off_4_channel_steps(gpu, monkeypatch):
    """A layer whose channels per tap are not a multiple of 4 does not take a
    forced thin configuration (a step would straddle two taps)."""
    from spinnv2_amd.runtime import Model

    monkeypatch.setenv("SPKV2_CONV_CFG", str(F32_THIN_CFGS[0]))
    g = models.single_conv(1, 6, 11, 13, 16, 3, 1, 1)
    blob = write_spk(g, "mi355x")
    xs = rng_inputs(g)
    with Model(blob) as m:
        m.set_input(0, xs[0])
        m.run()
        got = m.get_output(0)
        assert "thin" not in m.kernel_name(0)
    assert tnorm_err(got, run_oracle(blob, xs)[0]) <= FP32_TOL


@pytest.mark.parametrize("cfg", F32_IGEMM_CFGS)
def test_conv_hybrid_schedule(gpu, monkeypatch, cfg):
    """Hybrid schedule (whole tiles for a multiple of the CU count, the last
    n-tile columns split over k and summed by splitk_epilogue) on a layer
    with ragged M and N, bias, residual and Relu: against the oracle, and
    HIP-graph replays equal to the eager run."""
    from spinnv2_amd.runtime import Model

    monkeypatch.setenv("SPKV2_CONV_CFG", str(cfg))
    monkeypatch.setenv("SPKV2_CONV_HYBRID", "4")
    g = models.single_conv(4, 16, 63, 67, 200, 3, 1, 1, act="Relu", residual=True)
    blob = write_spk(g, "mi355x")
    xs = rng_inputs(g)
    with Model(blob) as m:
        for i, x in enumerate(xs):
            m.set_input(i, x)
        m.run()
        eager = m.get_output(0)
        name = m.kernel_name(0)
        m.set_graph_mode(True)
        for _ in range(2):
            for i, x in enumerate(xs):
                m.set_input(i, x)
            m.run()
            np.testing.assert_array_equal(m.get_output(0), eager)
    assert ",dp=" in name and "splitk=1," not in name, name
    want = run_oracle(blob, xs)[0]
    assert tnorm_err(eager, want) <= FP32_TOL


def test_split_k_graph_replays_match_eager(gpu, monkeypatch):
    """Split-K partials are fully rewritten by every run (no memset nodes in
    the captured graph), so its replays give the eager result every time."""
    from spinnv2_amd.runtime import Model

    monkeypatch.setenv("SPKV2_CONV_CFG", "7")  # 64x64x32 (the table's choice for the shape takes no split-K)
    monkeypatch.setenv("SPKV2_CONV_SPLITK", "6")
    g = models.single_conv(1, 256, 14, 14, 256, 3, 1, 1, act="Relu")
    blob = write_spk(g, "mi355x")
    xs = rng_inputs(g)
    with Model(blob) as m:
        m.set_input(0, xs[0])
        m.run()
        eager = m.get_output(0)
        assert "splitk=6" in m.kernel_name(0)
        m.set_graph_mode(True)
        for i in range(4):
            m.set_input(0, xs[0])
            m.run()
            np.testing.assert_array_equal(m.get_output(0), eager)
    want = run_oracle(blob, xs)[0]
    assert tnorm_err(eager, want) <= FP32_TOL


def _int8_network(depth=50, batch=2, image=32, profile="mi355x"):
    g = models.resnet(depth, batch, image=image, classes=10)
    xs = rng_inputs(g)
    cal = models.resnet(depth, 1, image=image, classes=10)
    samples = [models.make_input(cal.tensors[cal.inputs[0]].shape, 1000 + i) for i in range(4)]
    qp = calibrate_activation_scales(cal, samples) + quantize_conv_weights(g)
    return g, xs, write_spk(g, profile, quant_params=qp)


def test_int8_cpu_generic_package_runs_on_gpu(gpu):
    """An INT8 package as the reference compiler writes it for a CPU target:
    every conv under (simd, int8_im2col_gemm) with a (ref, reference)
    fallback (reference compiler/planner/kernel_spec.py:120-126) and the
    CPU scratch estimate.  It runs unchanged on the device int8 kernels:
    every conv's accumulators equal the oracle's, and the logits equal the
    mi355x package's bit for bit."""
    from oracle.spk_exec import OracleExecutor
    from spinnv2_amd.runtime import Model
    from spinnv2_amd.spk import format as F
    from spinnv2_amd.spk.kernel_spec import select_kernel_specs

    g, xs, blob = _int8_network(profile="cpu_generic")
    _, by_node, _ = select_kernel_specs(g, "cpu_generic")
    convs = [n for n in g.nodes if n.op_type == "Conv"]
    assert {(by_node[n.id].backend, F.KIND[by_node[n.id].kind]) for n in convs} == {("simd", 10)}
    _, _, blob_mi = _int8_network()
    ora = OracleExecutor(blob)
    want = ora.run(xs[0])[0].ravel()
    with Model(blob) as m:
        m.set_int8_capture(True)
        m.set_input(0, xs[0])
        m.run()
        got = m.get_output(0)
        for n in convs:
            np.testing.assert_array_equal(m.int8_accumulators(n.id, ora.acc[n.id].nbytes), ora.acc[n.id].ravel())
            assert m.kernel_name(n.id).startswith("conv_igemm_i8"), m.kernel_name(n.id)
    np.testing.assert_array_equal(got, run_gpu(blob_mi, xs)[0])
    assert tnorm_err(got, want) <= FP32_TOL


def test_gemm_trans_a_shapes(gpu):
    """Gemm with transA (A read as [K][rows], reference mm/gemm.c:17-31) at
    the FC shapes, alone and with transB and alpha."""
    for rows, k, nout, tb, alpha in [(1, 2048, 1000, 0, 1.0), (64, 2048, 1000, 1, 1.0), (7, 130, 33, 1, 0.5)]:
        g = models.single_gemm(rows, k, nout, trans_a=1, trans_b=tb, alpha=alpha)
        blob = write_spk(g, "mi355x")
        xs = rng_inputs(g)
        assert tnorm_err(run_gpu(blob, xs)[0], run_oracle(blob, xs)[0]) <= FP32_TOL, (rows, k, nout, tb)


def _int8_chain():
    """Bottleneck-style chain of int8 convs with no fp32 tail: 1x1 -> 3x3 ->
    1x1 + residual (also a graph output) -> 3x3 stride 2 -> 1x1."""
    from spinnv2_amd.spk.graph import Graph
    from spinnv2_amd.spk.passes import run_default_pipeline

    p = models.Params(3)
    g = Graph("i8chain")
    x = g.input("x", [2, 64, 14, 14])
    h = g.relu(g.conv(x, p.he((32, 64, 1, 1)), p.normal(32, 0.01)))
    h = g.relu(g.conv(h, p.he((32, 32, 3, 3)), p.normal(32, 0.01), pad=1))
    h3 = g.relu(g.add(g.conv(h, p.he((64, 32, 1, 1)), p.normal(64, 0.01)), x))
    h = g.relu(g.conv(h3, p.he((48, 64, 3, 3)), p.normal(48, 0.01), stride=2, pad=1))
    h = g.conv(h, p.he((40, 48, 1, 1)), None)
    g.mark_output(h)
    g.mark_output(h3)
    run_default_pipeline(g)
    xs = rng_inputs(g)
    samples = [[models.make_input([2, 64, 14, 14], 500 + i)] for i in range(3)]
    qp = calibrate_activation_scales(g, samples) + quantize_conv_weights(g)
    return g, xs, write_spk(g, "mi355x", quant_params=qp)


@pytest.mark.parametrize("handoff", ["1", "0"])
def test_int8_chain_bit_exact(gpu, monkeypatch, handoff):
    """Every conv int8; with handoff on, each conv whose only reader is the
    next int8 conv requantizes in its epilogue (the residual source, also a
    graph output, still writes fp32).  Outputs bit-exact either way."""
    from spinnv2_amd.runtime import Model

    monkeypatch.setenv("SPKV2_I8_HANDOFF", handoff)
    g, xs, blob = _int8_chain()
    want = run_oracle(blob, xs)
    with Model(blob) as m:
        m.set_input(0, xs[0])
        m.run()
        got = [m.get_output(0), m.get_output(1)]
        names = [m.kernel_name(n.id) for n in g.nodes if n.op_type == "Conv"]
    assert len(names) == 5 and all("conv_igemm_i8" in s for s in names)
    assert sum(",handoff" in s for s in names) == (4 if handoff == "1" else 0)
    for a_, b_ in zip(got, want):
        np.testing.assert_array_equal(a_.view(np.uint32), b_.view(np.uint32))


@pytest.mark.parametrize("mid", [45, 36])
def test_int8_handoff_odd_channels(gpu, mid):
    """Handoff into consumers whose padded channel stride is a multiple of
    16 with channels past M (45 -> 48: 16-byte stores, zero padding) or not
    (36: dword stores); bit-exact against the oracle."""
    from spinnv2_amd.spk.graph import Graph
    from spinnv2_amd.spk.passes import run_default_pipeline
    from spinnv2_amd.runtime import Model

    p = models.Params(8)
    g = Graph("i8odd")
    x = g.input("x", [2, 24, 13, 11])
    h = g.relu(g.conv(x, p.he((mid, 24, 1, 1)), p.normal(mid, 0.01)))
    h = g.relu(g.conv(h, p.he((20, mid, 3, 3)), p.normal(20, 0.01), pad=1))
    g.mark_output(g.conv(h, p.he((12, 20, 1, 1)), None))
    run_default_pipeline(g)
    xs = rng_inputs(g)
    qp = calibrate_activation_scales(g, [[models.make_input([2, 24, 13, 11], 800 + i)] for i in range(3)])
    blob = write_spk(g, "mi355x", quant_params=qp + quantize_conv_weights(g))
    want = run_oracle(blob, xs)[0]
    with Model(blob) as m:
        m.set_input(0, xs[0])
        m.run()
        got = m.get_output(0)
        names = [m.kernel_name(n.id) for n in g.nodes if n.op_type == "Conv"]
    assert sum(",handoff" in s for s in names) == 2, names
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))


def _int8_siblings():
    """One int8 conv whose output is read by three int8 convs: a 1x1 (takes
    the handoff), a 1x1 stride 2 (same quantization: shares that buffer) and
    a 3x3 pad 1 (another padded layout: quantizes for itself)."""
    from spinnv2_amd.spk.graph import Graph
    from spinnv2_amd.spk.passes import run_default_pipeline

    p = models.Params(5)
    g = Graph("i8siblings")
    x = g.input("x", [2, 48, 15, 13])
    h = g.relu(g.conv(x, p.he((64, 48, 1, 1)), p.normal(64, 0.01)))
    g.mark_output(g.conv(h, p.he((40, 64, 1, 1)), p.normal(40, 0.01)))
    g.mark_output(g.conv(h, p.he((72, 64, 1, 1)), None, stride=2))
    g.mark_output(g.conv(h, p.he((24, 64, 3, 3)), p.normal(24, 0.01), pad=1))
    run_default_pipeline(g)
    xs = rng_inputs(g)
    samples = [[models.make_input([2, 48, 15, 13], 600 + i)] for i in range(3)]
    qp = calibrate_activation_scales(g, samples) + quantize_conv_weights(g)
    return g, xs, write_spk(g, "mi355x", quant_params=qp)


@pytest.mark.parametrize("handoff", ["1", "0"])
def test_int8_shared_handoff_bit_exact(gpu, monkeypatch, handoff):
    """Two consumers read one handed-off int8 buffer; the third quantizes the
    fp32 tensor, which the producer therefore still writes.  Bit-exact
    against the oracle, and unchanged with a fault event armed (every tensor
    materialized)."""
    from spinnv2_amd.runtime import FaultEvent, Model

    monkeypatch.setenv("SPKV2_I8_HANDOFF", handoff)
    g, xs, blob = _int8_siblings()
    want = run_oracle(blob, xs)
    with Model(blob) as m:
        m.set_input(0, xs[0])
        m.run()
        got = [m.get_output(i) for i in range(3)]
        names = [m.kernel_name(n.id) for n in g.nodes if n.op_type == "Conv"]
        ev = FaultEvent(node_id=0, tensor_id=g.nodes[0].outputs[0], element_index=0, bit_index=0,
                        invocation_index=1000, seed=0, enabled=1)
        m.set_fault_event(ev)
        m.set_input(0, xs[0])
        m.run()
        armed = [m.get_output(i) for i in range(3)]
    assert len(names) == 4 and all("conv_igemm_i8" in s for s in names)
    if handoff == "1":
        assert [",handoff" in s for s in names] == [False, True, False, False], names
        assert [",shared" in s for s in names] == [False, False, True, False], names
    else:
        assert not any(",handoff" in s or ",shared" in s for s in names), names
    for a_, b_, c_ in zip(got, want, armed):
        np.testing.assert_array_equal(a_.view(np.uint32), b_.view(np.uint32))
        np.testing.assert_array_equal(c_.view(np.uint32), b_.view(np.uint32))


def test_int8_shared_handoff_skips_unread_fp32(gpu):
    """With only the two 1x1 consumers, every reader is served in int8: the
    producer's fp32 output is not written, and the results stay exact."""
    from spinnv2_amd.spk.graph import Graph
    from spinnv2_amd.spk.passes import run_default_pipeline
    from spinnv2_amd.runtime import Model

    p = models.Params(6)
    g = Graph("i8pair")
    x = g.input("x", [1, 32, 9, 11])
    h = g.relu(g.conv(x, p.he((64, 32, 3, 3)), p.normal(64, 0.01), pad=1))
    g.mark_output(g.conv(h, p.he((16, 64, 1, 1)), p.normal(16, 0.01)))
    g.mark_output(g.conv(h, p.he((16, 64, 1, 1)), p.normal(16, 0.01), stride=2))
    run_default_pipeline(g)
    xs = rng_inputs(g)
    qp = calibrate_activation_scales(g, [[models.make_input([1, 32, 9, 11], 700 + i)] for i in range(3)])
    blob = write_spk(g, "mi355x", quant_params=qp + quantize_conv_weights(g))
    want = run_oracle(blob, xs)
    from spinnv2_amd.spk import format as F

    h_id = g.nodes[0].outputs[0]
    with Model(blob) as m:
        lib = m.lib
        names = [m.kernel_name(n.id) for n in g.nodes if n.op_type == "Conv"]

        def span(tid):
            rec = F.TENSOR.unpack(ctypes.string_at(lib.spkv2_ctx_tensor_record(m.ctx, tid), F.TENSOR.size))
            return rec[14], rec[14] + rec[13]

        h0, h1 = span(h_id)
        others = [span(t) for t in [g.inputs[0]] + [n.outputs[0] for n in g.nodes[1:]]]
        assert all(e <= h0 or b >= h1 for b, e in others), "the plan places another tensor over h"
        sentinel = np.full((h1 - h0) // 4, 0x7FC00001, np.uint32)
        m.set_input(0, xs[0])
        m.run()
        got = [m.get_output(i) for i in range(2)]
        hptr = lib.spkv2_ctx_tensor_data(m.ctx, h_id)
        assert lib.spkv2_device_memcpy_h2d(hptr, sentinel.ctypes.data, sentinel.nbytes) == 0
        m.set_input(0, xs[0])
        m.run()
        again = [m.get_output(i) for i in range(2)]
        back = np.empty_like(sentinel)
        assert lib.spkv2_device_memcpy_d2h(back.ctypes.data, hptr, back.nbytes) == 0
    assert ",handoff" in names[1] and ",shared" in names[2], names
    for i, (a_, b_) in enumerate(zip(got, want)):
        np.testing.assert_array_equal(a_.view(np.uint32), b_.view(np.uint32), err_msg=f"output {i}")
    for i, (a_, b_) in enumerate(zip(again, want)):
        np.testing.assert_array_equal(a_.view(np.uint32), b_.view(np.uint32), err_msg=f"output {i}, second run")
    np.testing.assert_array_equal(back, sentinel)  # the fp32 tensor was not rewritten


def _int8_pool_consumers(shape, cout, third, pool_out):
    """int8 conv + Relu -> MaxPool 3x3/2 pad 1 -> a 1x1 int8 conv and a 1x1
    stride-2 int8 conv (the same quantization), plus `third`: None, or a 3x3
    pad-1 int8 conv (another padded layout, so it reads the fp32 tensor);
    pool_out also makes the pooled tensor a graph output."""
    from spinnv2_amd.spk.graph import Graph
    from spinnv2_amd.spk.passes import run_default_pipeline

    p = models.Params(9)
    g = Graph("i8pool")
    x = g.input("x", shape)
    h = g.relu(g.conv(x, p.he((cout, shape[1], 3, 3)), p.normal(cout, 0.01), pad=1))
    q = g.maxpool(h, 3, 2, 1)
    g.mark_output(g.conv(q, p.he((40, cout, 1, 1)), p.normal(40, 0.01)))
    g.mark_output(g.conv(q, p.he((24, cout, 1, 1)), None, stride=2))
    if third:
        g.mark_output(g.conv(q, p.he((16, cout, 3, 3)), p.normal(16, 0.01), pad=1))
    if pool_out:
        g.mark_output(q)
    run_default_pipeline(g)
    xs = rng_inputs(g)
    qp = calibrate_activation_scales(g, [[models.make_input(shape, 800 + i)] for i in range(3)])
    return g, xs, write_spk(g, "mi355x", quant_params=qp + quantize_conv_weights(g))


# (input shape, pooled channels, 3x3 reader, pooled tensor is an output):
# planes of 192 outputs (3 blocks of 64), 120 (a partial last block) and 32
# (less than one block); one and two 64-channel blocks
POOL_CASES = [([2, 16, 24, 32], 64, False, False), ([1, 16, 20, 24], 128, True, False),
              ([2, 8, 24, 32], 64, False, True), ([1, 8, 8, 16], 64, False, False)]


@pytest.mark.parametrize("handoff", ["1", "0"])
@pytest.mark.parametrize("case", range(len(POOL_CASES)))
def test_int8_maxpool_handoff_bit_exact(gpu, monkeypatch, case, handoff):
    """A MaxPool read by int8 convs quantizes its output for them in the
    pooling kernel (fp32 written only where something else reads it), and
    when only int8 convs read it, its producing int8 conv hands it int8 in
    turn: every output bit-exact against the oracle, eager and with a fault
    event armed (then the pool writes fp32 and each conv quantizes)."""
    from spinnv2_amd.runtime import FaultEvent, Model

    monkeypatch.setenv("SPKV2_I8_HANDOFF", handoff)
    shape, cout, third, pool_out = POOL_CASES[case]
    g, xs, blob = _int8_pool_consumers(shape, cout, third, pool_out)
    want = run_oracle(blob, xs)
    n_out = len(g.outputs)
    with Model(blob) as m:
        m.set_input(0, xs[0])
        m.run()
        got = [m.get_output(i) for i in range(n_out)]
        pool_name = [m.kernel_name(n.id) for n in g.nodes if n.op_type == "MaxPool"][0]
        names = [m.kernel_name(n.id) for n in g.nodes if n.op_type == "Conv"]
        m.set_input(0, xs[0])
        m.run()
        again = [m.get_output(i) for i in range(n_out)]
        ev = FaultEvent(node_id=0, tensor_id=g.nodes[0].outputs[0], element_index=0, bit_index=0,
                        invocation_index=1000, seed=0, enabled=1)
        m.set_fault_event(ev)
        m.set_input(0, xs[0])
        m.run()
        armed = [m.get_output(i) for i in range(n_out)]
    if handoff == "1":
        # with no fp32 reader of the pooled tensor, the first conv also hands
        # the pool its input in int8 (pooling quantized values)
        assert pool_name == ("maxpool3s2_q8+y" if third or pool_out else "maxpool3s2_i8"), pool_name
        assert ",handoff" in names[1] and ",shared" in names[2], names
    else:
        assert pool_name == "maxpool3s2_x4", pool_name
    for i, (a_, b_, c_, d_) in enumerate(zip(got, want, again, armed)):
        np.testing.assert_array_equal(a_.view(np.uint32), b_.view(np.uint32), err_msg=f"output {i}")
        np.testing.assert_array_equal(c_.view(np.uint32), b_.view(np.uint32), err_msg=f"output {i}, second run")
        np.testing.assert_array_equal(d_.view(np.uint32), b_.view(np.uint32), err_msg=f"output {i}, fault armed")


def test_int8_handoffs_off_after_registry_change(gpu):
    """A MaxPool kernel registered after prepare runs in place of the built-in
    pooling kernel, which alone writes the int8 handoff: the consumers then
    quantize the fp32 tensor the user kernel wrote (not a stale handoff
    buffer), and every output stays exact; after the registry is cleared the
    built-ins run without handoffs, still exact."""
    from spinnv2_amd.runtime import Model
    from spinnv2_amd.spk import format as F

    lib = gpu
    shape = [2, 8, 24, 32]
    g, xs, blob = _int8_pool_consumers(shape, 64, False, True)  # the pooled tensor is the last output
    xb = [models.make_input(shape, 4242)]
    want_a, want_b = run_oracle(blob, xs), run_oracle(blob, xb)
    pooled_b = np.ascontiguousarray(want_b[-1], np.float32)
    calls = []
    kernel_fn = ctypes.CFUNCTYPE(ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p)
    node_outputs = 4 + 2 * 4 + 8 * 4  # byte offset of outputs[0] in Spkv2NodeRecord

    def pool_b(ctx, node, scratch):
        calls.append(1)
        out = lib.spkv2_ctx_tensor_data(ctx, ctypes.c_uint32.from_address(node + node_outputs).value)
        return lib.spkv2_device_memcpy_h2d(out, pooled_b.ctypes.data, pooled_b.nbytes)

    k = kernel_fn(pool_b)
    n_out = len(g.outputs)
    try:
        with Model(blob) as m:
            m.set_input(0, xs[0])
            m.run()
            got_a = [m.get_output(i) for i in range(n_out)]
            assert m.kernel_name([n.id for n in g.nodes if n.op_type == "MaxPool"][0]) == "maxpool3s2_q8+y"
            assert lib.spkv2_register_kernel(F.OP["MaxPool"], F.BACKEND["mi355x"], F.KIND["device_elementwise"],
                                             ctypes.cast(k, ctypes.c_void_p), 0) == 0
            m.set_input(0, xb[0])
            m.run()
            got_b = [m.get_output(i) for i in range(n_out)]
            lib.spkv2_clear_user_kernels()
            m.set_input(0, xs[0])
            m.run()
            got_a2 = [m.get_output(i) for i in range(n_out)]
    finally:
        lib.spkv2_clear_user_kernels()
    assert len(calls) == 1
    for i in range(n_out):
        np.testing.assert_array_equal(got_a[i].view(np.uint32), want_a[i].view(np.uint32), err_msg=f"A {i}")
        np.testing.assert_array_equal(got_b[i].view(np.uint32), want_b[i].view(np.uint32), err_msg=f"B {i}")
        np.testing.assert_array_equal(got_a2[i].view(np.uint32), want_a[i].view(np.uint32), err_msg=f"A2 {i}")


@pytest.mark.parametrize("handoff", ["1", "0"])
def test_int8_resnet50_matches_oracle(gpu, monkeypatch, handoff):
    """A whole INT8 ResNet-50 (32x32 input), every conv int8: logits within
    the fp32 tolerance (the fp32 ReduceMean / Gemm tail sums in another
    order) and the same top-1."""
    from spinnv2_amd.runtime import Model

    monkeypatch.setenv("SPKV2_I8_HANDOFF", handoff)
    g, xs, blob = _int8_network()
    want = run_oracle(blob, xs)[0]
    with Model(blob) as m:
        m.set_input(0, xs[0])
        m.run()
        got = m.get_output(0)
    assert tnorm_err(got, want) <= FP32_TOL
    assert (got.reshape(2, -1).argmax(1) == want.reshape(2, -1).argmax(1)).all()


def test_int8_handoff_graph_mode_and_fault_path(gpu):
    """Graph replays of the handoff network equal eager; with a fault event
    armed (an injection on a node that never fires), every tensor is
    materialized and the result is unchanged."""
    from spinnv2_amd.runtime import FaultEvent, Model

    g, xs, blob = _int8_network(batch=1)
    with Model(blob) as m:
        m.set_input(0, xs[0])
        m.run()
        eager = m.get_output(0)
        m.set_graph_mode(True)
        for _ in range(3):
            m.set_input(0, xs[0])
            m.run()
            np.testing.assert_array_equal(m.get_output(0), eager)
        m.set_graph_mode(False)
        ev = FaultEvent(node_id=0, tensor_id=g.nodes[0].outputs[0], element_index=0, bit_index=0,
                        invocation_index=1000, seed=0, enabled=1)
        m.set_fault_event(ev)
        m.set_input(0, xs[0])
        m.run()
        np.testing.assert_array_equal(m.get_output(0), eager)


def test_fp32_pad_handoff_is_bit_identical(gpu, monkeypatch):
    """A 1x1 conv feeding a padded 3x3 conv stores straight into the 3x3
    conv's zero-padded input; outputs equal the unfused path bit for bit,
    and the oracle within tolerance (ResNet-50 at 64x64: every bottleneck)."""
    from spinnv2_amd.runtime import Model

    g = models.resnet(50, 2, image=64, classes=10)
    blob = write_spk(g, "mi355x")
    xs = rng_inputs(g)
    outs = {}
    for flag in ("1", "0"):
        monkeypatch.setenv("SPKV2_PAD_HANDOFF", flag)
        with Model(blob) as m:
            m.set_input(0, xs[0])
            m.run()
            outs[flag] = m.get_output(0)
            names = [m.kernel_name(n.id) for n in g.nodes if n.op_type == "Conv"]
        assert sum("+handoff" in s for s in names) == (16 if flag == "1" else 0)
    np.testing.assert_array_equal(outs["1"], outs["0"])
    assert tnorm_err(outs["1"], run_oracle(blob, xs)[0]) <= FP32_TOL


# Indexing / layout ops at larger sizes than the golden fixtures: bit-exact
# against the oracle (they move values without arithmetic).
INDEX_CASES = [
    ("Transpose", [2, 64, 40, 40], dict(perm=[0, 2, 3, 1])),
    ("Transpose", [1, 144, 8400], dict(perm=[0, 2, 1])),         # last two swapped: 32 x 32 LDS tiles
    ("Transpose", [2, 3, 45, 70], dict(perm=[0, 1, 3, 2])),      # ragged tiles, batch of 6
    ("Transpose", [2, 4, 8400], dict(perm=[0, 2, 1])),           # 4-row matrices
    ("Transpose", [2, 4, 16, 8400], dict(perm=[0, 2, 1, 3])),    # last axis kept: row copies, 16-byte
    ("Transpose", [3, 5, 7, 100], dict(perm=[2, 0, 1, 3])),
    ("Transpose", [2, 3, 130], dict(perm=[1, 0, 2])),            # rows of 130: scalar copies
    ("Tile", [1, 8, 1, 50], dict(reps=[2, 1, 30, 1])),
    ("Split", [1, 128, 40, 40], dict(sizes=[64, 64], axis=1)),
    ("Split", [1, 64, 8400], dict(sizes=[16, 16, 32], axis=1)),
    ("Slice", [1, 84, 8400], dict(start=4, end=84, axis=1, step=1)),
    ("Slice", [2, 33, 17], dict(start=-30, end=-1, axis=1, step=4)),
    # strided block copies: 16-byte path with several blocks, and odd widths (scalar path)
    ("Split", [4, 8, 6, 4], dict(sizes=[4, 4], axis=1)),
    ("Split", [2, 6, 5, 3], dict(sizes=[1, 5], axis=1)),
    ("Slice", [3, 10, 7], dict(start=2, end=9, axis=1, step=1)),
    ("Slice", [3, 16, 8], dict(start=4, end=12, axis=1, step=1)),
    ("Gather", [1, 8400, 4], dict(indices=list(range(8399, 0, -28)), axis=1)),
    ("GatherElements", [1, 8400, 6], dict(indices=np.random.default_rng(3).integers(0, 8400, (1, 300, 6)).tolist(), axis=1)),
    ("TopK", [1, 8400], dict(k=300, axis=-1, largest=1)),
    ("TopK", [4, 24000], dict(k=300, axis=1, largest=1)),
    ("TopK", [3, 1000, 5], dict(k=17, axis=1, largest=0)),
    ("TopK", [5, 130], dict(k=1, axis=1, largest=1)),
    ("TopK", [2, 70], dict(k=65, axis=-1, largest=0)),
    ("ReduceMax", [1, 80, 8400], dict(axes=[1], keepdims=0)),
    # the last axis: 16 lanes per row up to 128 (YOLO's 80 scores, ragged 7, the limit), a wave beyond
    ("ReduceMax", [2, 300, 80], dict(axes=[2], keepdims=0)),
    ("ReduceMax", [3, 33, 7], dict(axes=[2], keepdims=0)),
    ("ReduceMax", [2, 17, 128], dict(axes=[2], keepdims=0)),
    ("ReduceMax", [2, 17, 129], dict(axes=[2], keepdims=0)),
]


@pytest.mark.parametrize("batch,chans", [(3, (8, 16)), (2, (3, 5))])
def test_concat_strided_bitwise(gpu, batch, chans):
    """Channel Concat of batch > 1 inputs (one strided block copy per input:
    16-byte path for widths that allow it, scalar otherwise) against the
    oracle."""
    from spinnv2_amd.spk.graph import Graph

    g = Graph("concat")
    a = g.input("a", [batch, chans[0], 6, 10])
    b = g.input("b", [batch, chans[1], 6, 10])
    g.mark_output(g.concat([g.relu(a), g.relu(b)], axis=1))
    xs = rng_inputs(g)
    blob = write_spk(g, "mi355x")
    got = run_gpu(blob, xs)[0]
    want = run_oracle(blob, xs)[0]
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))


# TopK also on inputs rounded to a coarse grid, so values tie across the
# k-th place and the reference's heap history decides the selection, and on
# rows of one repeated value (a detector whose class scores all saturate to
# 1.0: the first k elements survive, no element enters the heap)
INDEX_RUNS = [(op, shape, kw, "normal") for op, shape, kw in INDEX_CASES] + \
    [(op, shape, kw, "ties") for op, shape, kw in INDEX_CASES if op == "TopK"] + \
    [(op, shape, kw, "const") for op, shape, kw in INDEX_CASES if op == "TopK"]


@pytest.mark.parametrize("op,shape,kw,dist", INDEX_RUNS,
                         ids=[f"{o}{i}_{d}" for i, (o, _, _, d) in enumerate(INDEX_RUNS)])
def test_index_ops_bitwise(gpu, op, shape, kw, dist):
    g = models.index_op(op, shape, **kw)
    xs = rng_inputs(g)
    if dist == "ties":
        xs = [np.round(x * 2).astype(np.float32) / 2 for x in xs]
    elif dist == "const":
        xs = [np.ones_like(x) for x in xs]
    got = run_gpu(write_spk(g, "mi355x"), xs, outputs=len(g.outputs))
    want = run_oracle(write_spk(g, "mi355x"), xs)
    for a_, b_ in zip(got, want):
        np.testing.assert_array_equal(a_.view(np.uint32), b_.view(np.uint32))


def test_yolo_v10n_640_e2e(gpu):
    """The YOLOv10n-style detector at 640x640 (8400 anchors, TopK 300): the
    whole graph -- C2f Split/Concat blocks, SPPF, PAN Resize/Concat, DFL
    Softmax, TopK, GatherElements -- on the device against the oracle."""
    from tests.helpers import check_detections

    g = models.yolo_v10n()
    blob = write_spk(g, "mi355x")
    xs = rng_inputs(g, dist="uniform")
    got = run_gpu(blob, xs, outputs=4)
    want = [np.asarray(o) for o in __import__("oracle.spk_exec", fromlist=["x"]).OracleExecutor(blob).run(*xs)]
    check_detections([a.reshape(w.shape) for a, w in zip(got, want)], want)


def test_yolo_v10n_graph_mode(gpu):
    from spinnv2_amd.runtime import Model

    g = models.yolo_v10n(image=320)
    blob = write_spk(g, "mi355x")
    xs = rng_inputs(g, dist="uniform")
    with Model(blob) as m:
        m.set_input(0, xs[0])
        m.run()
        eager = [m.get_output(i) for i in range(4)]
        m.set_graph_mode(True)
        for _ in range(3):
            m.set_input(0, xs[0])
            m.run()
            for i in range(4):
                np.testing.assert_array_equal(m.get_output(i), eager[i])


def test_fp32_pad_handoff_with_other_readers(gpu, monkeypatch):
    """A producer whose output feeds a padded conv and is also read elsewhere
    (here: a graph output and a Concat) writes both the padded copy and the
    tensor itself; every output matches the unfused path bit for bit."""
    from spinnv2_amd.runtime import Model
    from spinnv2_amd.spk.graph import Graph
    from spinnv2_amd.spk.passes import run_default_pipeline

    p = models.Params(5)
    g = Graph("handoff2")
    x = g.input("x", [1, 3, 40, 40])
    a = g.relu(g.conv(x, p.he((16, 3, 3, 3)), p.normal(16, 0.01), stride=2, pad=1))
    b = g.relu(g.conv(a, p.he((32, 16, 3, 3)), p.normal(32, 0.01), pad=1))
    c = g.concat([a, g.relu(g.conv(b, p.he((16, 32, 1, 1)), None))], axis=1)
    g.mark_output(a)
    g.mark_output(c)
    run_default_pipeline(g)
    blob = write_spk(g, "mi355x")
    xs = rng_inputs(g)
    outs = {}
    for flag in ("1", "0"):
        monkeypatch.setenv("SPKV2_PAD_HANDOFF", flag)
        with Model(blob) as m:
            m.set_input(0, xs[0])
            m.run()
            outs[flag] = [m.get_output(0), m.get_output(1)]
            if flag == "1":
                assert "+handoff" in m.kernel_name(1)
    for u, v in zip(outs["1"], outs["0"]):
        np.testing.assert_array_equal(u, v)
    for u, v in zip(outs["1"], run_oracle(blob, xs)):
        assert tnorm_err(u, v) <= FP32_TOL

