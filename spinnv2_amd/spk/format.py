"""SPK v0.3 binary layout: record structs and codes.

The package format is shared with the reference toolchain, so these layouts
and codes are necessarily identical to the reference
(runtime/include/spkv2_format.h:10-226; compiler/packager/spk_writer.py:17-106).
The mi355x backend and kernel kinds 12-15 are this backend's additions.
"""

from __future__ import annotations

import struct

MAGIC = 0x32564B50
VERSION_MAJOR = 0
VERSION_MINOR = 3

SECTION_METADATA = 1
SECTION_TARGET_PROFILE = 2
SECTION_TENSOR_TABLE = 3
SECTION_NODE_TABLE = 4
SECTION_ATTRIBUTES = 5
SECTION_WEIGHTS = 6
SECTION_MEMORY_PLAN = 7
SECTION_KERNEL_SPEC = 8
SECTION_QUANTIZATION = 9
SECTION_STRING_TABLE = 10
SECTION_DEBUG = 11
SECTION_CHECKSUM = 12
SECTION_PROTECTION_PLAN = 13

DTYPE = {"fp32": 1, "int8": 2, "fp16": 3}
DTYPE_NAME = {v: k for k, v in DTYPE.items()}
ROLE = {"input": 1, "output": 2, "weight": 3, "activation": 4, "constant": 5}
MEMORY_CLASS = {"INPUT": 1, "OUTPUT": 2, "WEIGHT": 3, "ACTIVATION_ARENA": 4, "EXTERNAL": 5}

OP = {
    "Add": 1, "Conv": 2, "Flatten": 3, "Gemm": 4, "MaxPool": 5, "Relu": 6, "Softmax": 7, "Mul": 8,
    "Sub": 9, "Div": 10, "Mod": 11, "Sigmoid": 12, "Reshape": 13, "Transpose": 14, "Concat": 15,
    "Split": 16, "ReduceMean": 17, "ReduceMax": 18, "MatMul": 19, "Resize": 20, "Tile": 21,
    "Unsqueeze": 22, "GatherElements": 23, "TopK": 24, "Cast": 25, "Slice": 26, "Gather": 27,
    "AveragePool": 28, "GlobalAveragePool": 29, "Clip": 30, "LeakyRelu": 31,
}
OP_NAME = {v: k for k, v in OP.items()}

BACKEND = {"ref": 1, "cpu": 2, "simd": 3, "delegate": 4, "mi355x": 5}
KIND = {
    "reference": 1, "direct": 2, "im2col_gemm": 3, "packed_gemm": 4, "pointwise_1x1": 5,
    "depthwise_direct": 6, "winograd_3x3s1": 7, "conv3x3s2_direct": 8, "winograd_f43": 9,
    "int8_im2col_gemm": 10, "bnns_fp32": 11,
    # mi355x target
    "implicit_gemm_f32": 12, "implicit_gemm_i8": 13, "gemm_f32": 14, "device_elementwise": 15,
}
ACTIVATION = {None: 0, "Relu": 1, "Silu": 2}
QUANT_SCHEME = {"per_tensor": 1, "per_channel": 2}
NO_SPEC = 0xFFFFFFFF

HEADER = struct.Struct("<IHHHHIIIIIIQQQII")          # 68 B
SECTION = struct.Struct("<IIQQII")                  # 32 B
TENSOR = struct.Struct("<IHHHH8IQQII")              # 68 B
NODE = struct.Struct("<IHHHH8I4IIIII")              # 76 B
ATTR = struct.Struct("<Iiii4i2i2i2i2i2fii8i3i")     # 124 B
MEMORY_PLAN = struct.Struct("<IHHIQQII")            # 36 B
KERNEL_SPEC = struct.Struct("<IIHHHHHHQQII")        # 44 B
QUANT_PARAM = struct.Struct("<IHHIQ")               # 20 B
PROTECTION = struct.Struct("<IIHHffQ")              # 28 B

assert (HEADER.size, SECTION.size, TENSOR.size, NODE.size, ATTR.size, MEMORY_PLAN.size,
        KERNEL_SPEC.size, QUANT_PARAM.size, PROTECTION.size) == (68, 32, 68, 76, 124, 36, 44, 20, 28)


def fnv1a32(data: bytes | bytearray | memoryview) -> int:
    """FNV-1a 32-bit, the package checksum (reference loader.c:25-32).

    Large packages are hashed by the runtime library's exported
    spkv2_fnv1a32 (the function its loader verifies with); a pure-Python loop
    covers small blobs and hosts where the library is not built.
    """
    data = bytes(data)
    if len(data) > (1 << 16):
        lib = _native()
        if lib is not None:
            return int(lib.spkv2_fnv1a32(data, len(data)))
    h = 2166136261
    for b in data:
        h ^= b
        h = (h * 16777619) & 0xFFFFFFFF
    return h


_LIB = None


def _native():
    global _LIB
    if _LIB is None:
        import ctypes
        from pathlib import Path

        path = Path(__file__).resolve().parent.parent / "lib" / "libspkv2_mi355x.so"
        try:
            lib = ctypes.CDLL(str(path))
            lib.spkv2_fnv1a32.restype = ctypes.c_uint32
            lib.spkv2_fnv1a32.argtypes = [ctypes.c_char_p, ctypes.c_size_t]
            _LIB = lib
        except OSError:
            _LIB = False
    return _LIB or None
