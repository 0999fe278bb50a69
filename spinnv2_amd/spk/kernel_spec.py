"""KernelSpec selection per target profile.

`cpu_generic` / `cpu_generic_nobnns` / `cpu_ref` reproduce the reference's
choice of (backend, kind) for those profiles (compiler/planner/kernel_spec.py:
71-224, compiler/target/profiles/cpu_generic.json), including its per-node
scratch estimate (kernel_spec.py:240-298), so the reference runtime runs the
packages as it would run its own compiler's output.

`mi355x` is this backend's target: fp32 Conv -> (mi355x, implicit_gemm_f32)
with fallback (mi355x, reference) [the direct device conv]; INT8 Conv ->
(mi355x, implicit_gemm_i8); Gemm / MatMul -> (mi355x, gemm_f32); every other
op -> (mi355x, device_elementwise).  Fallbacks never name a CPU kind.
"""

from __future__ import annotations

from dataclasses import dataclass

from .graph import Graph, Node

SIMD_TILE_BYTES = 32 * 1024 * 1024
SIMD_REF_OPS = {"Add", "Mul", "Sub", "Div", "Relu", "Sigmoid", "Transpose", "ReduceMax", "ReduceMean", "Softmax",
                "MaxPool", "Resize", "AveragePool", "GlobalAveragePool", "Clip", "LeakyRelu"}

PROFILES = {
    "mi355x": {"name": "mi355x", "backends": ["mi355x"], "scratch_arena_max": 1 << 30,
               "activation_arena_max": 0},
    "cpu_generic": {"name": "cpu_generic", "backends": ["ref", "cpu", "simd"], "bnns": True,
                    "scratch_arena_max": 33554432, "activation_arena_max": 0},
    "cpu_generic_nobnns": {"name": "cpu_generic_nobnns", "backends": ["ref", "cpu", "simd"], "bnns": False,
                           "scratch_arena_max": 1 << 30, "activation_arena_max": 0},
    "cpu_ref": {"name": "cpu_ref", "backends": ["ref"], "scratch_arena_max": 1 << 30, "activation_arena_max": 0},
}


@dataclass
class Spec:
    id: int
    node_id: int
    kind: str
    backend: str
    dtype: str = "fp32"
    scratch_bytes: int = 0
    fallback: int = 0xFFFFFFFF


def _align(v: int, a: int = 16) -> int:
    return (v + a - 1) // a * a


def _conv_geometry(g: Graph, n: Node):
    x = g.tensors[n.inputs[0]].shape
    w = g.tensors[n.inputs[1]].shape
    y = g.tensors[n.outputs[0]].shape
    return x, w, y


def _cpu_scratch(g: Graph, n: Node, kind: str, backend: str) -> int:
    """reference kernel_spec.py:240-298"""
    if n.op_type != "Conv" or kind in ("pointwise_1x1", "depthwise_direct", "conv3x3s2_direct", "bnns_fp32",
                                       "reference"):
        return 0
    x, w, y = _conv_geometry(g, n)
    if kind == "int8_im2col_gemm":
        k = x[1] * w[2] * w[3]
        spatial = y[2] * y[3]
        return _align(x[1] * x[2] * x[3] + k * spatial + w[0] * spatial * 4)
    if kind == "im2col_gemm":
        k = x[1] * w[2] * w[3]
        if backend == "simd":
            return _align(min(k * y[2] * y[3] * 4, 2 * 1024 * 1024))
        return _align(k * 4)
    return 0


def _cpu_generic_conv_kind(g: Graph, n: Node, bnns: bool) -> str:
    """reference kernel_spec.py:146-224 with the cpu_generic token list."""
    x, w, y = _conv_geometry(g, n)
    group = int(n.attrs.get("group", 1))
    strides = list(n.attrs.get("strides", [1, 1]))
    pads = list(n.attrs.get("pads", [0, 0, 0, 0]))
    dil = list(n.attrs.get("dilations", [1, 1]))
    if bnns and group == 1:
        return "bnns_fp32"
    if group == 1 and w[2] == 1 and w[3] == 1 and strides == [1, 1] and pads == [0, 0, 0, 0] and dil == [1, 1]:
        return "pointwise_1x1"
    if group == x[1] and group == w[0] and w[2] == 3 and w[3] == 3 and dil == [1, 1]:
        return "depthwise_direct"
    return "im2col_gemm"


def select_kernel_specs(g: Graph, profile: str) -> tuple[list[Spec], dict[int, Spec], int]:
    prof = PROFILES[profile]
    specs: list[Spec] = []
    by_node: dict[int, Spec] = {}
    scratch = 0

    def add(spec: Spec) -> Spec:
        spec.id = len(specs)
        specs.append(spec)
        return spec

    for n in g.nodes:
        if profile == "mi355x":
            if n.op_type == "Conv":
                int8 = g.tensors[n.inputs[1]].dtype == "int8"
                sel = add(Spec(0, n.id, "implicit_gemm_i8" if int8 else "implicit_gemm_f32", "mi355x",
                               "int8" if int8 else "fp32"))
                if not int8:
                    sel.fallback = add(Spec(0, n.id, "reference", "mi355x")).id
            elif n.op_type in ("Gemm", "MatMul"):
                sel = add(Spec(0, n.id, "gemm_f32", "mi355x"))
            else:
                sel = add(Spec(0, n.id, "device_elementwise", "mi355x"))
        elif profile == "cpu_ref":
            sel = add(Spec(0, n.id, "reference", "ref"))
        else:
            ref = Spec(0, n.id, "reference", "ref")
            if n.op_type == "Conv":
                int8 = g.tensors[n.inputs[1]].dtype == "int8"
                if int8 and int(n.attrs.get("group", 1)) == 1:
                    sel = Spec(0, n.id, "int8_im2col_gemm", "simd", "int8")
                else:
                    sel = Spec(0, n.id, _cpu_generic_conv_kind(g, n, prof.get("bnns", True)), "simd")
            elif n.op_type in ("Gemm", "MatMul"):
                sel = Spec(0, n.id, "direct", "simd")
            elif n.op_type in SIMD_REF_OPS:
                sel = Spec(0, n.id, "reference", "simd")
            else:
                sel = ref
            sel.scratch_bytes = _cpu_scratch(g, n, sel.kind, sel.backend)
            add(sel)
            if sel is not ref:
                sel.fallback = add(ref).id
        by_node[n.id] = sel
        scratch = max(scratch, sel.scratch_bytes)
    if scratch > prof["scratch_arena_max"]:
        raise MemoryError(f"scratch arena {scratch} exceeds profile limit {prof['scratch_arena_max']}")
    return specs, by_node, scratch
