"""The C-ABI library on the CPU: it loads, exports every entry point that
include/*.h declares, rejects malformed packages with the reference loader's
error codes, keeps the reference's kernel-registration limits, and fails
loudly (never falls back to the CPU) when no GPU is present.  No GPU.
"""

from __future__ import annotations

import ctypes
import re
import struct
from pathlib import Path

import pytest

from spinnv2_amd.runtime import SIGNATURES, device_available, load_library
from spinnv2_amd.spk import format as F
from spinnv2_amd.spk import models, write_spk

ROOT = Path(__file__).resolve().parent.parent
DECL = re.compile(r"\b(spkv2_[a-z0-9_]+)\s*\(")


def declared_symbols() -> set[str]:
    names = set()
    for h in sorted((ROOT / "include").glob("*.h")):
        text = h.read_text()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        text = re.sub(r"//[^\n]*", "", text)
        names |= set(DECL.findall(text))
    return names


def test_headers_declare_the_reference_api():
    names = declared_symbols()
    # runtime/include/spkv2_runtime.h:25-79 of the reference
    for ref_name in ("spkv2_load_file", "spkv2_load_memory", "spkv2_prepare", "spkv2_prepare_with_scratch",
                     "spkv2_set_input", "spkv2_bind_input", "spkv2_bind_output", "spkv2_get_output",
                     "spkv2_get_output_size", "spkv2_run", "spkv2_free", "spkv2_register_kernel",
                     "spkv2_clear_user_kernels", "spkv2_set_fault_event", "spkv2_clear_fault_event",
                     "spkv2_get_reliability_stats", "spkv2_reset_reliability_stats", "spkv2_get_range_observation",
                     "spkv2_reset_range_observations", "spkv2_profile_dump", "spkv2_runtime_version"):
        assert ref_name in names, ref_name


def test_library_exports_every_declared_symbol():
    lib = load_library()
    missing = [n for n in sorted(declared_symbols()) if not hasattr(lib, n)]
    assert not missing, missing


def test_ctypes_binding_covers_every_declared_symbol():
    assert set(SIGNATURES) == declared_symbols()


def test_runtime_version():
    assert load_library().spkv2_runtime_version().decode().startswith("0.3")


@pytest.mark.parametrize("data,want", [(b"", 0x811C9DC5), (b"a", 0xE40C292C), (b"foobar", 0xBF9CF968)])
def test_fnv1a32_known_answers(data, want):
    # published FNV-1a 32-bit test vectors
    assert load_library().spkv2_fnv1a32(data, len(data)) == want


# ---------------------------------------------------------------- loading

def _load(blob: bytes) -> tuple[int, ctypes.c_void_p]:
    lib = load_library()
    buf = ctypes.create_string_buffer(blob, len(blob))
    ctx = ctypes.c_void_p()
    rc = lib.spkv2_load_memory(buf, len(blob), ctypes.byref(ctx))
    if rc == 0:
        lib.spkv2_free(ctx)
    return rc, buf


@pytest.fixture(scope="module")
def lenet_blob() -> bytes:
    return write_spk(models.lenet(), "mi355x")


def _sections(blob: bytes):
    hdr = F.HEADER.unpack_from(blob, 0)
    hsize, count = hdr[4], hdr[5]
    return [(hsize + i * F.SECTION.size, F.SECTION.unpack_from(blob, hsize + i * F.SECTION.size))
            for i in range(count)]


def _patch_section_kind(blob: bytes, kind: int, new_kind: int) -> bytes:
    b = bytearray(blob)
    for off, sec in _sections(blob):
        if sec[0] == kind:
            struct.pack_into("<I", b, off, new_kind)
    return bytes(b)


def test_load_valid_package(lenet_blob):
    assert _load(lenet_blob)[0] == 0


def test_load_error_codes(lenet_blob):
    """Return codes of the reference loader (runtime/core/loader.c:140-206)."""
    assert _load(lenet_blob[:40])[0] == -1                          # shorter than the header
    bad = bytearray(lenet_blob)
    bad[0] ^= 0xFF
    assert _load(bytes(bad))[0] == -2                               # magic
    bad = bytearray(lenet_blob)
    struct.pack_into("<H", bad, 4, 7)
    assert _load(bytes(bad))[0] == -2                               # version_major
    bad = bytearray(lenet_blob)
    struct.pack_into("<I", bad, 12, 1 << 20)
    assert _load(bytes(bad))[0] == -3                               # section directory past the end
    bad = bytearray(lenet_blob)
    off = _sections(lenet_blob)[0][0]
    struct.pack_into("<Q", bad, off + 8, len(lenet_blob))           # section offset past the end
    assert _load(bytes(bad))[0] == -3
    assert _load(_patch_section_kind(lenet_blob, F.SECTION_TENSOR_TABLE, F.SECTION_DEBUG))[0] == -4
    assert _load(_patch_section_kind(lenet_blob, F.SECTION_WEIGHTS, F.SECTION_DEBUG))[0] == -4
    assert _load(_patch_section_kind(lenet_blob, F.SECTION_CHECKSUM, F.SECTION_DEBUG))[0] == -5
    bad = bytearray(lenet_blob)
    wsec = [s for _, s in _sections(lenet_blob) if s[0] == F.SECTION_WEIGHTS][0]
    bad[wsec[2] + 5] ^= 0x01                                        # one weight bit
    assert _load(bytes(bad))[0] == -6


def test_load_file_roundtrip(tmp_path, lenet_blob):
    lib = load_library()
    p = tmp_path / "lenet.spk"
    p.write_bytes(lenet_blob)
    ctx = ctypes.c_void_p()
    assert lib.spkv2_load_file(str(p).encode(), ctypes.byref(ctx)) == 0
    size = ctypes.c_size_t()
    assert lib.spkv2_get_output_size(ctx, 0, ctypes.byref(size)) == 0
    assert size.value == 10 * 4
    lib.spkv2_free(ctx)
    assert lib.spkv2_load_file(str(tmp_path / "missing.spk").encode(), ctypes.byref(ctx)) == -1


# ---------------------------------------------------------- kernel registry

KERNEL_FN = ctypes.CFUNCTYPE(ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p)


@pytest.fixture()
def noop_kernel():
    fn = KERNEL_FN(lambda ctx, node, scratch: 0)
    yield fn
    load_library().spkv2_clear_user_kernels()


def test_register_kernel_limits(noop_kernel):
    """reference runtime/tests/test_register_kernel.c:133-146: 64 user
    kernels fit, the 65th is refused with -2; a null function is -1."""
    lib = load_library()
    lib.spkv2_clear_user_kernels()
    ptr = ctypes.cast(noop_kernel, ctypes.c_void_p)
    assert lib.spkv2_register_kernel(F.OP["Relu"], 0, 0, None, 0) == -1
    for i in range(64):
        assert lib.spkv2_register_kernel(F.OP["Relu"], 0, i, ptr, 0) == 0
    assert lib.spkv2_register_kernel(F.OP["Relu"], 0, 64, ptr, 0) == -2
    lib.spkv2_clear_user_kernels()
    assert lib.spkv2_register_kernel(F.OP["Relu"], 0, 0, ptr, 0) == 0


# ------------------------------------------------------------- no device

@pytest.mark.skipif(device_available(), reason="checks the behaviour without a GPU")
def test_prepare_without_gpu_fails_loudly(lenet_blob):
    lib = load_library()
    buf = ctypes.create_string_buffer(lenet_blob, len(lenet_blob))
    ctx = ctypes.c_void_p()
    assert lib.spkv2_load_memory(buf, len(lenet_blob), ctypes.byref(ctx)) == 0
    assert lib.spkv2_prepare(ctx, None, 0) == -30
    assert b"device" in lib.spkv2_mi355x_last_error()
    assert lib.spkv2_run(ctx) != 0
    lib.spkv2_free(ctx)


def test_missing_library_raises(tmp_path):
    with pytest.raises(RuntimeError, match="not built"):
        load_library(tmp_path / "libspkv2_mi355x.so")
