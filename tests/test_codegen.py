"""Static C wrappers generated from mi355x packages (the reference's
compiler/codegen/c_codegen.py API on top of libspkv2_mi355x).

CPU: the generator's header macros, checksums and external-weight split; the
generated C compiles with gcc against include/ and the built runtime, and
its exported entry points answer argument errors without a GPU.  GPU: the
LeNet wrappers compiled by __graft_entry__.build() (embedded and external
weights) run through ctypes and match the CPU oracle, from host buffers and
from device-resident ones.
"""

from __future__ import annotations

import ctypes
import re
import subprocess

import numpy as np
import pytest

from spinnv2_amd import codegen
from spinnv2_amd.spk import format as F
from spinnv2_amd.spk import models, write_spk

from .helpers import FP32_TOL, rng_inputs, run_oracle, tnorm_err


def lenet_blob() -> bytes:
    return write_spk(models.lenet(), "mi355x")


def macros(text: str) -> dict[str, str]:
    return dict(re.findall(r"#define (\w+) (.+)", text))


def test_header_describes_the_package(tmp_path):
    g = models.lenet()
    blob = write_spk(g, "mi355x")
    files = codegen.generate_c_from_spk(blob, tmp_path, name="lenet-1")
    sym = "lenet_1"
    assert files["header"] == tmp_path / f"{sym}.h"
    m = macros(files["header"].read_text())
    assert m[f"{sym.upper()}_INPUT_SIZE_0"] == f"((size_t){g.tensors[g.inputs[0]].size_bytes}u)"
    assert m[f"{sym.upper()}_OUTPUT_SIZE_0"] == f"((size_t){g.tensors[g.outputs[0]].size_bytes}u)"
    assert m[f"{sym.upper()}_SPK_CHECKSUM"] == f"0x{F.fnv1a32(blob):08x}u"
    assert codegen.sanitize("9net") == "m_9net"


def test_external_weights_split(tmp_path):
    blob = lenet_blob()
    files = codegen.generate_c_from_spk(blob, tmp_path, name="lenet_ext", external_weights=True)
    info = codegen.inspect_spk(blob)
    weights = files["weights"].read_bytes()
    assert weights == blob[info.weights_offset:info.weights_offset + info.weights_size]
    zeroed = bytearray(blob)
    zeroed[info.weights_offset:info.weights_offset + info.weights_size] = bytes(info.weights_size)
    m = macros(files["header"].read_text())
    assert m["LENET_EXT_SPK_CHECKSUM"] == f"0x{F.fnv1a32(bytes(zeroed)):08x}u"
    assert "int lenet_ext_init(const char *weights_path);" in files["header"].read_text()


def test_generated_c_compiles_and_checks_arguments(tmp_path, lib):
    blob = lenet_blob()
    codegen.generate_c_from_spk(blob, tmp_path, name="lenet")
    subprocess.run(["make", "-s", "-C", str(tmp_path)], check=True)
    w = ctypes.CDLL(str(tmp_path / "liblenet.so"))
    vp = ctypes.c_void_p
    w.lenet_verify_checksum.argtypes = [ctypes.c_char_p, ctypes.c_size_t]
    assert w.lenet_verify_checksum(blob, len(blob)) == 0
    assert w.lenet_verify_checksum(blob[:-1], len(blob) - 1) == -2
    w.lenet_run.argtypes = [vp, vp]
    x = np.zeros(28 * 28, np.float32)
    y = np.zeros(10, np.float32)
    assert w.lenet_run(x.ctypes.data, y.ctypes.data) == -3          # not initialised
    w.lenet_run_checked.argtypes = [vp, ctypes.c_size_t, vp, ctypes.c_size_t]
    assert w.lenet_run_checked(x.ctypes.data, 4 * 783, y.ctypes.data, 40) == -2


def _load_example(name: str):
    lib = codegen.EXAMPLE_DIR / name / f"lib{name}.so"
    if not lib.exists():
        pytest.fail(f"{lib} missing: __graft_entry__.build() compiles the generated examples")
    w = ctypes.CDLL(str(lib))
    vp = ctypes.c_void_p
    # attribute access caches the function object (indexing makes a new one
    # each time, without these argtypes)
    getattr(w, f"{name}_run").argtypes = [vp, vp]
    getattr(w, f"{name}_run_device").argtypes = [ctypes.POINTER(vp), ctypes.c_int, ctypes.POINTER(vp), ctypes.c_int]
    getattr(w, f"{name}_free").restype = None
    return w


@pytest.mark.gpu
@pytest.mark.parametrize("name", ["lenet", "lenet_ext"])
def test_gpu_generated_wrapper_runs_lenet(gpu, name):
    from spinnv2_amd.runtime import DeviceBuffer

    print(f"[codegen] {name}", flush=True)
    g = models.lenet()
    blob = write_spk(g, "mi355x")
    xs = rng_inputs(g, seed=3, dist="uniform")
    want = run_oracle(blob, xs)[0]
    w = _load_example(name)
    if name == "lenet_ext":
        w.lenet_ext_init.argtypes = [ctypes.c_char_p]
        assert w.lenet_ext_init(str(codegen.EXAMPLE_DIR / name / "missing.bin").encode()) == -20
        rc = w.lenet_ext_init(str(codegen.EXAMPLE_DIR / name / f"{name}_weights.bin").encode())
    else:
        rc = w.lenet_init()
    assert rc == 0
    try:
        x = np.ascontiguousarray(xs[0], np.float32)
        y = np.zeros(want.size, np.float32)
        assert getattr(w, f"{name}_run")(x.ctypes.data, y.ctypes.data) == 0
        assert tnorm_err(y, want) <= FP32_TOL and int(y.argmax()) == int(want.argmax())
        dx, dy = DeviceBuffer(x.nbytes), DeviceBuffer(y.nbytes)
        try:
            dx.upload(x)
            ins = (ctypes.c_void_p * 1)(dx.ptr.value)
            outs = (ctypes.c_void_p * 1)(dy.ptr.value)
            assert getattr(w, f"{name}_run_device")(ins, 1, outs, 1) == 0
            np.testing.assert_array_equal(dy.download(), y)
        finally:
            dx.free()
            dy.free()
    finally:
        getattr(w, f"{name}_free")()
