"""GPU parity on the benchmark configurations at their stated sizes.

ResNet-18 fp32 at 224x224, batch 32, and the INT8 ResNet-50 at 224x224,
batch 1 and batch 64 (BASELINE configs[1] and [4]), against the CPU oracle
through the C ABI.  Reference semantics: runtime/kernels/reference/conv/conv.c
for fp32, runtime/kernels/optimized/conv/conv_int8.c:121-210 for INT8.

Bars: fp32 tensor-normalized max error <= 1e-4 with the same top-1; INT8
int32 accumulators of every conv node bit-exact; INT8 logits (which pass
through the fp32 ReduceMean / Gemm tail) within 1e-4 with the same top-1.
"""

from __future__ import annotations

import numpy as np
import pytest

from spinnv2_amd.spk import models, write_spk
from spinnv2_amd.spk.quantize import calibrate_activation_scales, quantize_conv_weights

from .helpers import FP32_TOL, rng_inputs, run_gpu, run_oracle, tnorm_err

pytestmark = pytest.mark.gpu


def test_resnet18_224_b32_images_match_batch1(gpu):
    """ResNet-18 at batch 32: every image is independent through every node,
    so images 0 and 31 of the batch must agree with batch-1 runs of the same
    images (other tiles and split-K choices: within the fp32 tolerance), and
    image 0 with the oracle."""
    g32 = models.resnet(18, 32)
    x = rng_inputs(g32)[0]
    print("resnet18 b=32", flush=True)
    out32 = run_gpu(write_spk(g32, "mi355x"), [x])[0].reshape(32, -1)
    blob1 = write_spk(models.resnet(18, 1), "mi355x")
    for i in (0, 31):
        one = run_gpu(blob1, [x[i:i + 1]])[0]
        assert tnorm_err(out32[i], one) <= FP32_TOL, i
        assert np.argmax(out32[i]) == np.argmax(one), i
    want0 = run_oracle(blob1, [x[0:1]])[0]
    assert tnorm_err(out32[0], want0) <= FP32_TOL
    assert np.argmax(out32[0]) == np.argmax(want0)


_CAL = {}


def _int8_scales():
    """Activation scales as the benchmark makes them: 16 seeded single-image
    calibration batches through the fp32 forward of the fused graph."""
    if "act" not in _CAL:
        g1 = models.resnet(50, 1)
        samples = [models.make_input(g1.tensors[g1.inputs[0]].shape, 1000 + i) for i in range(16)]
        _CAL["act"] = calibrate_activation_scales(g1, samples)
    return _CAL["act"]


def _int8_resnet50(batch):
    g = models.resnet(50, batch)
    return g, write_spk(g, "mi355x", quant_params=quantize_conv_weights(g) + _int8_scales())


@pytest.mark.parametrize("handoff", ["1", "0"])
def test_int8_resnet50_224_b1_every_accumulator(gpu, monkeypatch, handoff):
    """INT8 ResNet-50 at 224x224, batch 1: the raw int32 accumulators of all
    53 conv nodes, captured during the network run itself (so from the
    inputs the handoffs delivered), equal the oracle's bit for bit; the
    logits are within the fp32 tolerance with the same top-1."""
    from oracle.spk_exec import OracleExecutor
    from spinnv2_amd.runtime import Model

    monkeypatch.setenv("SPKV2_I8_HANDOFF", handoff)
    g, blob = _int8_resnet50(1)
    x = rng_inputs(g)[0]
    ora = OracleExecutor(blob)
    want = ora.run(x)[0].ravel()
    convs = [n for n in g.nodes if n.op_type == "Conv"]
    assert len(convs) == 53 and set(ora.acc) == {n.id for n in convs}
    print(f"int8 resnet50 224 b=1 handoff={handoff}", flush=True)
    with Model(blob) as m:
        m.set_int8_capture(True)
        m.set_input(0, x)
        m.run()
        got = m.get_output(0)
        names = [m.kernel_name(n.id) for n in convs]
        for n in convs:
            acc = m.int8_accumulators(n.id, ora.acc[n.id].nbytes)
            np.testing.assert_array_equal(acc, ora.acc[n.id].ravel(), err_msg=f"node {n.id} {m.kernel_name(n.id)}")
    assert all(s.startswith("conv_igemm_i8") for s in names), names
    assert (sum(",handoff" in s for s in names) > 0) == (handoff == "1")
    assert tnorm_err(got, want) <= FP32_TOL
    assert np.argmax(got) == np.argmax(want)


def test_int8_resnet50_224_b64_images_match_batch1(gpu):
    """INT8 ResNet-50 at 224x224, batch 64 (the benchmark workload): the
    reference quantizes each image on its own (conv_int8.c:121-140), so
    images 0 and 63 of the batch must give the batch-1 logits (the fp32
    Gemm tail may sum in another order: within tolerance) with the same
    top-1, and image 0 the oracle's."""
    g64, blob64 = _int8_resnet50(64)
    x = rng_inputs(g64)[0]
    print("int8 resnet50 224 b=64", flush=True)
    out64 = run_gpu(blob64, [x])[0].reshape(64, -1)
    _, blob1 = _int8_resnet50(1)
    for i in (0, 63):
        one = run_gpu(blob1, [x[i:i + 1]])[0]
        assert tnorm_err(out64[i], one) <= FP32_TOL, i
        assert np.argmax(out64[i]) == np.argmax(one), i
    want0 = run_oracle(blob1, [x[0:1]])[0]
    assert tnorm_err(out64[0], want0) <= FP32_TOL
    assert np.argmax(out64[0]) == np.argmax(want0)


def test_int8_capture_graph_mode(gpu):
    """Accumulator capture is re-recorded into the HIP graph: replays give the
    eager accumulators and outputs."""
    from spinnv2_amd.runtime import Model

    from .test_gpu_parity import _int8_network

    g, xs, blob = _int8_network(batch=1)
    conv0 = [n for n in g.nodes if n.op_type == "Conv"][-1]
    nbytes = 4 * int(np.prod(g.shape(conv0.outputs[0])))
    with Model(blob) as m:
        m.set_input(0, xs[0])
        m.run()
        out = m.get_output(0)
        m.set_graph_mode(True)
        m.set_input(0, xs[0])
        m.run()
        m.set_int8_capture(True)
        for _ in range(2):
            m.set_input(0, xs[0])
            m.run()
            np.testing.assert_array_equal(m.get_output(0), out)
            acc = m.int8_accumulators(conv0.id, nbytes)
        m.set_graph_mode(False)
        m.set_input(0, xs[0])
        m.run()
        np.testing.assert_array_equal(m.int8_accumulators(conv0.id, nbytes), acc)
        assert np.any(acc != 0)
