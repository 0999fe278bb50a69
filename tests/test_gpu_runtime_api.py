"""The runtime API's own contracts on the device, as the reference's C tests
state them for the CPU runtime: kernel registration and dispatch
(runtime/tests/test_register_kernel.c), caller arenas
(runtime/tests/test_prepare_arena.c), bind / get sizes and codes
(runtime/core/executor.c:249-324).
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest

from spinnv2_amd.spk import format as F
from spinnv2_amd.spk import models, write_spk

pytestmark = pytest.mark.gpu

KERNEL_FN = ctypes.CFUNCTYPE(ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p)
NODE_OUTPUTS = F.NODE.size - 4 * 4 - 4 * 4  # byte offset of outputs[0] in Spkv2NodeRecord


def _fill_kernel(lib, value: float, rc: int = 0):
    """A user kernel that writes `value` into the node's output through the
    device accessors (what a third-party kernel does), or returns `rc`."""

    def fn(ctx, node, scratch):
        if rc != 0:
            return rc
        out_id = ctypes.c_uint32.from_address(node + NODE_OUTPUTS).value
        rec = lib.spkv2_ctx_tensor_record(ctx, out_id)
        size = F.TENSOR.unpack(ctypes.string_at(rec, F.TENSOR.size))[13]
        host = np.full(size // 4, value, np.float32)
        return lib.spkv2_device_memcpy_h2d(lib.spkv2_ctx_tensor_data(ctx, out_id), host.ctypes.data, size)

    return KERNEL_FN(fn)


@pytest.fixture()
def relu_pkg():
    g = models.single_op("Relu", [1, 1, 1, 4])
    return write_spk(g, "mi355x")


def _run(blob, x):
    from spinnv2_amd.runtime import Model

    with Model(blob) as m:
        m.set_input(0, x)
        m.run()
        return m.get_output(0)


def test_node_record_layout():
    # outputs[0] follows id, op, flags, counts and inputs[8]
    assert NODE_OUTPUTS == 4 + 2 * 4 + 8 * 4


def test_user_kernel_overrides_and_clear_restores(gpu, relu_pkg):
    """test_register_kernel.c:40-103: a registered kernel replaces the
    built-in, the higher priority of two wins, clearing restores the
    built-in."""
    lib = gpu
    x = np.array([[[[-1, 0, 1, 2]]]], np.float32)
    backend, kind = F.BACKEND["mi355x"], F.KIND["device_elementwise"]
    k42, k99 = _fill_kernel(lib, 42.0), _fill_kernel(lib, 99.0)
    try:
        lib.spkv2_clear_user_kernels()
        assert lib.spkv2_register_kernel(F.OP["Relu"], backend, kind, ctypes.cast(k42, ctypes.c_void_p), 10) == 0
        np.testing.assert_array_equal(_run(relu_pkg, x), [42, 42, 42, 42])
        assert lib.spkv2_register_kernel(F.OP["Relu"], backend, kind, ctypes.cast(k99, ctypes.c_void_p), 50) == 0
        np.testing.assert_array_equal(_run(relu_pkg, x), [99, 99, 99, 99])
        lib.spkv2_clear_user_kernels()
        np.testing.assert_array_equal(_run(relu_pkg, x), [0, 0, 1, 2])
    finally:
        lib.spkv2_clear_user_kernels()


def test_unsupported_user_kernel_falls_back(gpu, relu_pkg):
    """A kernel answering -99 hands the node to the next candidate
    (reference runtime/kernels/reference/kernels.c:201-245)."""
    lib = gpu
    x = np.array([[[[-3, -0.5, 0.5, 3]]]], np.float32)
    k = _fill_kernel(lib, 0.0, rc=-99)
    try:
        lib.spkv2_clear_user_kernels()
        assert lib.spkv2_register_kernel(F.OP["Relu"], F.BACKEND["mi355x"], F.KIND["device_elementwise"],
                                         ctypes.cast(k, ctypes.c_void_p), 100) == 0
        np.testing.assert_array_equal(_run(relu_pkg, x), [0, 0, 0.5, 3])
    finally:
        lib.spkv2_clear_user_kernels()


def test_caller_arena(gpu):
    """test_prepare_arena.c: an arena smaller than the header's activation
    arena is refused with -2; one of the exact size is used as given."""
    from spinnv2_amd.runtime import DeviceBuffer, Model

    g = models.lenet()
    blob = write_spk(g, "mi355x")
    need = F.HEADER.unpack_from(blob, 0)[12]
    x = models.make_input(g.tensors[g.inputs[0]].shape, 3, "uniform")
    want = _run(blob, x)
    small, exact = DeviceBuffer(8), DeviceBuffer(need)
    try:
        m = Model(blob, prepare=False)
        try:
            assert m.lib.spkv2_prepare(m.ctx, small.ptr, 8) == -2
            assert m.lib.spkv2_prepare(m.ctx, exact.ptr, need) == 0
            m.set_input(0, x)
            m.run()
            np.testing.assert_array_equal(m.get_output(0), want)
        finally:
            m.close()
    finally:
        small.free()
        exact.free()


def test_io_size_and_index_codes(gpu):
    """executor.c:249-324: a wrong size is -2, an unknown index fails, and
    bound device buffers are used in place."""
    from spinnv2_amd.runtime import DeviceBuffer, Model

    g = models.lenet()
    blob = write_spk(g, "mi355x")
    x = models.make_input(g.tensors[g.inputs[0]].shape, 5, "uniform")
    with Model(blob) as m:
        lib = m.lib
        assert lib.spkv2_set_input(m.ctx, 0, x.ctypes.data, x.nbytes - 4) == -2
        assert lib.spkv2_set_input(m.ctx, 1, x.ctypes.data, x.nbytes) != 0
        y = np.empty(10, np.float32)
        assert lib.spkv2_get_output(m.ctx, 0, y.ctypes.data, y.nbytes + 4) == -2
        assert lib.spkv2_get_output(m.ctx, 3, y.ctypes.data, y.nbytes) != 0
        m.set_input(0, x)
        m.run()
        want = m.get_output(0)
        xb, yb = DeviceBuffer(x.nbytes), DeviceBuffer(y.nbytes)
        try:
            xb.upload(x)
            assert lib.spkv2_bind_input(m.ctx, 0, xb.ptr, x.nbytes - 4) == -2
            m.bind_input(0, xb)
            m.bind_output(0, yb)
            m.run()
            np.testing.assert_array_equal(yb.download(), want)
        finally:
            xb.free()
            yb.free()


def test_conv_over_2gib_is_refused(gpu):
    """A conv whose fp32 input or output reaches 2 GiB is refused at prepare
    (SPKV2_E_UNSUPPORTED, -32) instead of overflowing 32-bit byte offsets."""
    from spinnv2_amd.runtime import Model, RuntimeError_

    g = models.single_conv(1, 8, 8192, 8200, 8, 1, 1, 0)  # 537M elements per tensor: 2.1 GB
    blob = write_spk(g, "mi355x")
    with pytest.raises(RuntimeError_) as e:
        Model(blob)
    assert e.value.code == -32


def test_user_conv_kernel_before_prepare_then_cleared(gpu):
    """A user Conv kernel registered before prepare wins the conv nodes; the
    built-in plans are prepared anyway (apart from the user's node_cache
    slot), so when the user kernel answers -99 the built-in runs the node,
    and after the registry is cleared the built-ins run every node: both
    equal the oracle.  No handoff is set up with a node a user kernel runs."""
    from spinnv2_amd.runtime import Model
    from tests.helpers import FP32_TOL, rng_inputs, run_oracle, tnorm_err

    lib = gpu
    g = models.resnet(50, 1, image=64, classes=10)
    blob = write_spk(g, "mi355x")
    xs = rng_inputs(g)
    want = run_oracle(blob, xs)[0]
    calls = []
    objects = {}

    def refuse(ctx, node, scratch):
        calls.append(1)
        # the user owns the ABI node_cache slot: keep an object of its own
        # there (freed by the runtime with spkv2_platform_free, no destructor)
        slot = ctypes.c_void_p()
        nid = ctypes.c_uint32.from_address(node).value
        assert lib.spkv2_ctx_node_cache(ctx, nid, ctypes.addressof(slot), None) == 0
        if not ctypes.c_void_p.from_address(slot.value).value:
            obj = lib.spkv2_platform_malloc(64)
            ctypes.memset(obj, 0x5A, 64)
            ctypes.c_void_p.from_address(slot.value).value = obj
            objects[nid] = obj
        return -99

    k = KERNEL_FN(refuse)
    try:
        lib.spkv2_clear_user_kernels()
        assert lib.spkv2_register_kernel(F.OP["Conv"], F.BACKEND["mi355x"], F.KIND["implicit_gemm_f32"],
                                         ctypes.cast(k, ctypes.c_void_p), 5) == 0
        with Model(blob) as m:
            names = [m.kernel_name(n.id) for n in g.nodes if n.op_type == "Conv"]
            assert not any("+handoff" in s for s in names), names
            for mode in (False, True):
                m.set_graph_mode(mode)
                m.set_input(0, xs[0])
                m.run()
                assert tnorm_err(m.get_output(0), want) <= FP32_TOL
            assert len(calls) == 2 * len(names)
            lib.spkv2_clear_user_kernels()
            for mode in (False, True):
                m.set_graph_mode(mode)
                m.set_input(0, xs[0])
                m.run()
                assert tnorm_err(m.get_output(0), want) <= FP32_TOL
            assert len(calls) == 2 * len(names)
            # the slots still hold the user's objects, untouched by the built-ins
            assert len(objects) == len(names)
            for nid, obj in objects.items():
                slot = ctypes.c_void_p()
                assert lib.spkv2_ctx_node_cache(m.ctx, nid, ctypes.addressof(slot), None) == 0
                assert ctypes.c_void_p.from_address(slot.value).value == obj
                assert ctypes.string_at(obj, 64) == b"\x5a" * 64
    finally:
        lib.spkv2_clear_user_kernels()


def test_register_then_clear_restores_handoffs_and_graph(gpu):
    """Registering a kernel for an op no node uses leaves every node's kernel
    as at prepare: handoffs and HIP-graph replay stay on, bit-identical to
    before; a MaxPool kernel that does take a node turns them off until the
    registry is cleared again."""
    from spinnv2_amd.runtime import Model
    from tests.helpers import rng_inputs

    lib = gpu
    g = models.resnet(50, 2, image=64, classes=10)
    blob = write_spk(g, "mi355x")
    xs = rng_inputs(g)
    k = _fill_kernel(lib, 7.0)
    try:
        lib.spkv2_clear_user_kernels()
        with Model(blob) as m:
            m.set_graph_mode(True)
            m.set_input(0, xs[0])
            m.run()
            base = m.get_output(0)
            assert lib.spkv2_register_kernel(F.OP["TopK"], F.BACKEND["mi355x"], F.KIND["device_elementwise"],
                                             ctypes.cast(k, ctypes.c_void_p), 0) == 0
            m.set_input(0, xs[0])
            m.run()
            np.testing.assert_array_equal(m.get_output(0), base)
            assert lib.spkv2_register_kernel(F.OP["MaxPool"], F.BACKEND["mi355x"], F.KIND["device_elementwise"],
                                             ctypes.cast(k, ctypes.c_void_p), 0) == 0
            m.set_input(0, xs[0])
            m.run()
            assert not np.array_equal(m.get_output(0), base)  # the pooled tensor is all 7.0 now
            lib.spkv2_clear_user_kernels()
            for _ in range(2):
                m.set_input(0, xs[0])
                m.run()
                np.testing.assert_array_equal(m.get_output(0), base)
    finally:
        lib.spkv2_clear_user_kernels()
