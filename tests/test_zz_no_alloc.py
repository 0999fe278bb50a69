"""The allocation-free INT8 accumulator entry point
(spkv2_mi355x_conv_int8_accumulators_noalloc) against the allocating one
(spkv2_mi355x_conv_int8_accumulators) and the oracle, through the C ABI:
two calls in a row on one GPU, the second with a smaller input (the shared
staging array keeps the first call's larger contents), with and without
split-K, and a size beyond the 16 MiB array refused with a clear error."""

from __future__ import annotations

import numpy as np
import pytest

from spinnv2_amd.spk import models, write_spk
from spinnv2_amd.spk.quantize import calibrate_activation_scales, quantize_conv_weights

from .helpers import rng_inputs

pytestmark = pytest.mark.gpu


def _package(g):
    xs = rng_inputs(g)
    qp = calibrate_activation_scales(g, [xs]) + quantize_conv_weights(g)
    return xs, write_spk(g, "mi355x", quant_params=qp)


@pytest.mark.parametrize("split", ["1", "3"])
def test_noalloc_accumulators_match_allocating_entry_point(gpu, monkeypatch, split):
    from oracle.spk_exec import OracleExecutor
    from spinnv2_amd.runtime import Model

    monkeypatch.setenv("SPKV2_I8_SPLITK", split)
    lib = gpu
    graphs = [models.single_conv(4, 64, 28, 28, 96, 3, 1, 1, act="Relu", residual=True),  # 1.2 MB of int32
              models.single_conv(1, 32, 9, 11, 40, 1, 1, 0, act=None)]                    # 16 KB: smaller
    for k, g in enumerate(graphs):
        xs, blob = _package(g)
        ora = OracleExecutor(blob)
        ora.run(*xs)
        nid = [n.id for n in g.nodes if n.op_type == "Conv"][0]
        size = ora.acc[nid].nbytes
        print(f"[noalloc] split={split} conv {g.shape(g.nodes[nid].outputs[0])} {size} B", flush=True)
        with Model(blob) as m:
            for i, x in enumerate(xs):
                m.set_input(i, x)
            m.run()
            if k == 0:  # the second conv has a single k-tile, which never splits
                assert f"splitk={split}" in m.kernel_name(nid), m.kernel_name(nid)
            want = m.int8_accumulators(nid, size)
            got = np.full(size // 4, -7, np.int32)
            assert lib.spkv2_mi355x_conv_int8_accumulators_noalloc(m.ctx, nid, got.ctypes.data, size) == 0
        np.testing.assert_array_equal(got, want)
        np.testing.assert_array_equal(got, ora.acc[nid].ravel())


def test_noalloc_accumulators_refuse_more_than_the_array(gpu):
    from spinnv2_amd.runtime import Model

    lib = gpu
    g = models.single_conv(21, 64, 56, 56, 64, 1, 1, 0, act=None)  # 21*64*56*56*4 B > 16 MiB
    xs, blob = _package(g)
    size = 21 * 64 * 56 * 56 * 4
    assert size > 16 << 20
    with Model(blob) as m:
        m.set_input(0, xs[0])
        m.run()
        out = np.empty(size // 4, np.int32)
        assert lib.spkv2_mi355x_conv_int8_accumulators_noalloc(m.ctx, 0, out.ctypes.data, size) == -32
        assert b"16 MiB" in lib.spkv2_mi355x_last_error()
