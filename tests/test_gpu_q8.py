"""GPU parity of the INT8 configuration with int8 tensors between nodes
(per-channel symmetric int8 weights, per-tensor
asymmetric activations from min/max calibration, int32 accumulation,
fixed-point requantization with round-half-away, fused Relu clamp).

The reference runtime has no such mode, so the checker is the oracle's
restatement (oracle/spk_oracle.c, oracle_q8_*), pinned on the CPU by
tests/test_oracle_q8.py.  The bar is the north star's for INT8: the int32
accumulators and the requantized int8 outputs bit-exact, here for every
int8 tensor of the network (read back from the device), and the dequantized
spatial mean (an exact integer sum and two IEEE double operations) bit-exact.
"""

from __future__ import annotations

import numpy as np
import pytest

from spinnv2_amd.spk import models, write_spk
from spinnv2_amd.spk.graph import Graph
from spinnv2_amd.spk.passes import run_default_pipeline
from spinnv2_amd.spk.quantize import quantize_int8_activations

from .helpers import FP32_TOL, rng_inputs, tnorm_err

pytestmark = pytest.mark.gpu


def _q8_package(g: Graph, n_cal: int = 4, mark=()):
    """Calibrates on seeded samples and writes the mode's package; `mark`
    lists extra tensors to make graph outputs before quantization."""
    for t in mark:
        g.mark_output(t)
    samples = [[models.make_input(g.tensors[t].shape, 1000 + i + 7 * k) for k, t in enumerate(g.inputs)]
               for i in range(n_cal)]
    qp = quantize_int8_activations(g, samples)
    return write_spk(g, "mi355x", quant_params=qp)


def _int8_tensors(g: Graph) -> list[int]:
    return [t.id for t in g.tensors if t.dtype == "int8" and t.role == "activation"]


def _check_all(g: Graph, blob: bytes, xs, *, graph_mode=False, capture=True, exact_outputs=None):
    """Runs the package on the GPU and the oracle; every int8 tensor and
    every conv's accumulators bit-exact; `exact_outputs` lists the graph
    outputs that must be bit-exact (the rest: the fp32 tolerance)."""
    from oracle.spk_exec import OracleExecutor
    from spinnv2_amd.runtime import Model

    ora = OracleExecutor(blob)
    vals = ora.run(*xs, keep=True)
    convs = [n for n in g.nodes if n.op_type == "Conv"]
    q8 = _int8_tensors(g)
    assert q8, "no int8 tensor in the package"
    with Model(blob) as m:
        if capture:
            m.set_int8_capture(True)
        m.set_graph_mode(graph_mode)
        for _ in range(2 if graph_mode else 1):
            for i, x in enumerate(xs):
                m.set_input(i, x)
            m.run()
        names = [m.kernel_name(n.id) for n in convs]
        for t in q8:
            got = m.read_int8_tensor(t, g.tensors[t].shape)
            np.testing.assert_array_equal(got, vals[t], err_msg=f"int8 tensor {t}")
        if capture:
            for n in convs:
                acc = m.int8_accumulators(n.id, ora.acc[n.id].nbytes)
                np.testing.assert_array_equal(acc, ora.acc[n.id].ravel(), err_msg=f"node {n.id} {m.kernel_name(n.id)}")
        outs = [m.get_output(i) for i in range(len(g.outputs))]
    for i, t in enumerate(g.outputs):
        want = np.asarray(vals[t], np.float32).ravel()
        if exact_outputs is not None and i in exact_outputs:
            np.testing.assert_array_equal(outs[i].view(np.uint32), want.view(np.uint32), err_msg=f"output {i}")
        else:
            assert tnorm_err(outs[i], want) <= FP32_TOL, i
    assert all(s.startswith("conv_igemm_q8") for s in names), names
    return names


def _chain(batch=2, c=16, hw=9, widths=(24, 40), k=3, stride=1, residual=True, relu_last=True, pool=False,
           in_ch=3, k0=3):
    """fp32 input -> conv k0 x k0 (quantized on load) -> [MaxPool] -> conv
    k x k -> conv 1x1 (+ residual from the first conv's branch) ->
    ReduceMean."""
    p = models.Params(17)
    g = Graph("q8_chain")
    x = g.input("x", [batch, in_ch, hw, hw])
    a = g.relu(g.conv(x, p.he((c, in_ch, k0, k0)), p.normal(c, 0.05), pad=k0 // 2))
    if pool:
        a = g.maxpool(a, *(pool if isinstance(pool, tuple) else (3, 2, 1)))
    b = g.relu(g.conv(a, p.he((widths[0], c, k, k)), p.normal(widths[0], 0.05), stride=stride, pad=k // 2))
    y = g.conv(b, p.he((widths[1], widths[0], 1, 1)), p.normal(widths[1], 0.05))
    if residual:
        r = g.conv(a, p.he((widths[1], c, 1, 1)), p.normal(widths[1], 0.05), stride=stride)
        y = g.add(y, r)
    if relu_last:
        y = g.relu(y)
    h = g.reduce_mean(y, [2, 3], keepdims=1)
    g.mark_output(g.flatten(h, 1))
    run_default_pipeline(g)
    return g


CHAINS = [
    dict(),
    dict(batch=1, hw=7, k=1),
    dict(batch=3, c=32, hw=12, stride=2),
    dict(batch=2, hw=11, pool=True, residual=False),
    dict(batch=1, c=20, hw=10, widths=(36, 52), relu_last=False),
    dict(batch=2, hw=8, k=5),
    dict(batch=2, hw=40, k=1, residual=False),  # a 40 x 40 spatial mean: 25 pixels per lane
    dict(batch=2, hw=12, pool=(2, 2, 0), residual=False),  # a 2 x 2 window: the generic pooling loop
]


@pytest.mark.parametrize("case", range(len(CHAINS)))
def test_q8_chain_bit_exact(gpu, case):
    g = _chain(**CHAINS[case])
    blob = _q8_package(g)
    print(f"[q8] chain {CHAINS[case]}", flush=True)
    _check_all(g, blob, rng_inputs(g), exact_outputs={0})


# tile configurations of conv_i8.hip's table: LDS-staged, pixel-gather and
# direct-weight kernels (each with and without split-K) and the persistent
# direct-weight kernels (whole tiles), on a chain whose 3x3
# layer reads a halo; 64-channel tensors so that the pixel-gather kernels
# with 64-byte k-tiles can read every layer
Q8_FORCED = [(c, s) for c in (2, 5, 9, 12, 18, 19, 20, 21, 31, 33) for s in (1, 3)] + \
            [(c, 1) for c in (23, 24, 25, 26, 29, 35)]


@pytest.mark.parametrize("cfg,split", Q8_FORCED, ids=[f"q8cfg{c}_split{s}" for c, s in Q8_FORCED])
def test_q8_every_tile_config_and_split(gpu, monkeypatch, cfg, split):
    from spinnv2_amd.runtime import RuntimeError_

    monkeypatch.setenv("SPKV2_I8_CFG", str(cfg))
    monkeypatch.setenv("SPKV2_I8_SPLITK", str(split))
    g = _chain(batch=2, c=64, hw=10, widths=(64, 64), in_ch=64, k0=1)
    blob = _q8_package(g)
    print(f"[q8] forced cfg {cfg} split {split}", flush=True)
    names = _check_all(g, blob, rng_inputs(g), exact_outputs={0})
    assert any(f"splitk={split}" in n for n in names) or split == 1, names


def test_q8_graph_mode_and_capture(gpu):
    g = _chain(batch=2, hw=9, pool=True)
    blob = _q8_package(g)
    _check_all(g, blob, rng_inputs(g), graph_mode=True, exact_outputs={0})


def _q8_resnet50(batch, n_cal=16):
    """ResNet-50 224x224 in the mode, calibrated as bench.py does: 16 seeded
    single-image batches through the batch-1 fp32 graph (the same weights);
    the ReduceMean output is a second graph output."""
    g = models.resnet(50, batch)
    g.mark_output([n for n in g.nodes if n.op_type == "ReduceMean"][0].outputs[0])
    cal = models.resnet(50, 1)
    samples = [models.make_input(cal.tensors[cal.inputs[0]].shape, 1000 + i) for i in range(n_cal)]
    qp = quantize_int8_activations(g, samples, calibrate_on=cal)
    return g, write_spk(g, "mi355x", quant_params=qp)


def test_q8_resnet50_224_b1_every_int8_tensor(gpu):
    """ResNet-50 224x224, batch 1: all 54 int8 tensors, all 53 convs'
    accumulators and the ReduceMean output bit-exact; the logits (fp32 Gemm)
    within tolerance."""
    g, blob = _q8_resnet50(1)
    assert len(_int8_tensors(g)) == 54
    print("[q8] resnet50 224 b=1", flush=True)
    _check_all(g, blob, rng_inputs(g), exact_outputs={1})


def test_q8_resnet50_224_b64_images_equal_batch1_oracle(gpu):
    """The benchmark workload: ResNet-50 224x224 batch 64 in this mode.
    Images 0 and 63: every int8 tensor and every conv's accumulators equal
    the oracle's batch-1 values for that image, and the ReduceMean rows bit
    for bit; graph replay equals eager."""
    from oracle.spk_exec import OracleExecutor
    from spinnv2_amd.runtime import Model

    g64, blob64 = _q8_resnet50(64)
    g1, blob1 = _q8_resnet50(1)
    rm = g64.outputs[1]
    x = rng_inputs(g64)[0]
    want = {}
    for i in (0, 63):
        ora = OracleExecutor(blob1)
        want[i] = (ora.run(x[i:i + 1], keep=True), ora.acc)
    q8 = _int8_tensors(g64)
    convs = [n for n in g64.nodes if n.op_type == "Conv"]
    print("[q8] resnet50 224 b=64", flush=True)
    with Model(blob64) as m:
        m.set_int8_capture(True)
        m.set_input(0, x)
        m.run()
        eager = m.get_output(1)
        for t in q8:
            got = m.read_int8_tensor(t, g64.tensors[t].shape)
            for i in (0, 63):
                np.testing.assert_array_equal(got[i], want[i][0][t][0], err_msg=f"tensor {t} image {i}")
        for n in convs:
            shape = g64.shape(n.outputs[0])
            acc = m.int8_accumulators(n.id, 4 * int(np.prod(shape))).reshape(shape)
            for i in (0, 63):
                np.testing.assert_array_equal(acc[i], want[i][1][n.id][0], err_msg=f"node {n.id} image {i}")
        mean = eager.reshape(64, -1)
        for i in (0, 63):
            w = np.asarray(want[i][0][rm], np.float32).ravel()
            np.testing.assert_array_equal(mean[i].view(np.uint32), w.view(np.uint32))
        m.set_int8_capture(False)
        m.set_graph_mode(True)
        for _ in range(3):
            m.set_input(0, x)
            m.run()
            np.testing.assert_array_equal(m.get_output(1).view(np.uint32), eager.view(np.uint32))


def test_q8_refuses_user_kernels_and_protection_on_int8_tensors(gpu, monkeypatch):
    """Nodes that read or write int8 tensors between nodes run only on the
    built-in kernels that hold those tensors' device buffers.  A user kernel
    registered for them after prepare makes spkv2_run refuse (-32) without
    calling it, and clearing the registry restores the bit-identical run;
    registered before prepare, prepare refuses.  A protection plan naming an
    int8 tensor (its guards read fp32 tensors) is refused at prepare (this
    repository's writer never writes one; the package here is forced)."""
    import ctypes

    from spinnv2_amd.runtime import Model, RuntimeError_, load_library
    from spinnv2_amd.spk import format as F
    from spinnv2_amd.spk import writer
    from spinnv2_amd.spk.writer import Protection

    lib = load_library()
    g = _chain()
    blob = _q8_package(g)
    xs = rng_inputs(g)
    calls = []
    kernel = ctypes.CFUNCTYPE(ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p)(
        lambda ctx, node, scratch: calls.append(1) or -99)
    register = lambda: lib.spkv2_register_kernel(F.OP["Conv"], F.BACKEND["mi355x"], F.KIND["implicit_gemm_i8"],
                                                 ctypes.cast(kernel, ctypes.c_void_p), 5)
    try:
        lib.spkv2_clear_user_kernels()
        with Model(blob) as m:
            m.set_input(0, xs[0])
            m.run()
            base = m.get_output(0)
            assert register() == 0
            m.set_input(0, xs[0])
            assert m.run_rc() == -32 and not calls
            lib.spkv2_clear_user_kernels()
            # the memory plan may reuse the input's arena region once its
            # last reader ran: inputs are set before every run
            m.set_input(0, xs[0])
            m.run()
            np.testing.assert_array_equal(m.get_output(0).view(np.uint32), base.view(np.uint32))
        assert register() == 0
        m = Model(blob, prepare=False)
        try:
            with pytest.raises(RuntimeError_) as err:
                m.prepare()
            assert err.value.code == -32 and not calls
        finally:
            m.close()
    finally:
        lib.spkv2_clear_user_kernels()
    # a range guard on a conv whose output is an int8 tensor
    h = _chain()
    conv = next(n for n in h.nodes if n.op_type == "Conv")
    samples = [[models.make_input(h.tensors[h.inputs[0]].shape, 1000 + i)] for i in range(4)]
    qp = quantize_int8_activations(h, samples)
    t = h.tensors[conv.outputs[0]]
    assert t.dtype == "int8"
    strict = writer._protection_section

    def forced(g_, entries, offset):  # the writer's own check refuses int8 outputs
        t.dtype = "fp32"
        try:
            return strict(g_, entries, offset)
        finally:
            t.dtype = "int8"

    monkeypatch.setattr(writer, "_protection_section", forced)
    prot = write_spk(h, "mi355x", quant_params=qp, protection=[Protection(conv.id, "range_guard_rerun", -1e3, 1e3)])
    m = Model(prot, prepare=False)
    try:
        with pytest.raises(RuntimeError_) as err:
            m.prepare()
        assert err.value.code == -32
    finally:
        m.close()


def test_q8_resnet18_basic_blocks(gpu):
    """ResNet-18's basic blocks in the mode (3x3 convs carrying the residual,
    1x1 stride-2 projections, the 7x7 stem and its MaxPool) at 64x64, batch
    2: every int8 tensor and every conv's accumulators bit-exact; the spatial
    mean (a second graph output) bit-exact, the logits within tolerance."""
    g = models.resnet(18, 2, image=64)
    blob = _q8_package(g, mark=[[n for n in g.nodes if n.op_type == "ReduceMean"][0].outputs[0]])
    assert len(_int8_tensors(g)) == 21  # 20 conv outputs and the stem MaxPool's
    _check_all(g, blob, rng_inputs(g), exact_outputs={1})
