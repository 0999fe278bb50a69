"""KernelSpec selection per target profile.

`cpu_generic` / `cpu_generic_nobnns` / `cpu_ref` / `cpu_arm_neon` reproduce
the reference's choice of (backend, kind) for those profiles
(compiler/planner/kernel_spec.py:71-224, compiler/target/profiles/*.json),
including its per-node scratch estimate (kernel_spec.py:240-298), so the
reference runtime runs the packages as it would run its own compiler's
output.  `cpu_arm_neon_exp` selects the two conv kinds the reference runtime
dispatches but no reference profile emits (Winograd F(2,3), 3x3/s2 direct),
so that packages carrying every conv kind code can be produced.

`mi355x` is this backend's target, described by profiles/mi355x.json in the
reference's profile schema (compiler/target/profiles/cpu_generic.json): each
op lists `mi355x_<kind>` tokens in preference order, the first that applies
wins, the next one becomes the fallback spec (reference kernel_spec.py:71-144
does the same with its simd tokens).  fp32 / fp16-weight Conv ->
(mi355x, implicit_gemm_f32) with fallback (mi355x, reference) [the direct
device conv]; INT8 Conv -> (mi355x, implicit_gemm_i8); Gemm / MatMul ->
(mi355x, gemm_f32); every other op -> (mi355x, device_elementwise).
Fallbacks never name a CPU kind.

The mi355x kinds carry their device workspace in the spec's scratch_bytes:
the zero-padded input copy (fp32 NCHW, or quantized int8 NHWC) plus room for
split-K partial sums, so the runtime runs them out of the package's scratch
arena (a caller-provided one under spkv2_prepare_with_scratch) instead of
allocating.
"""

from __future__ import annotations

import json
from dataclasses import dataclass
from pathlib import Path

from .graph import Graph, Node, conv_out

SIMD_TILE_BYTES = 32 * 1024 * 1024
SIMD_REF_OPS = {"Add", "Mul", "Sub", "Div", "Relu", "Sigmoid", "Transpose", "ReduceMax", "ReduceMean", "Softmax",
                "MaxPool", "Resize", "AveragePool", "GlobalAveragePool", "Clip", "LeakyRelu"}

MI355X_PROFILE = json.loads((Path(__file__).resolve().parent / "profiles" / "mi355x.json").read_text())

# split-K bound the device workspace estimate allows for: the runtime's
# largest split, capped per node (a plan that needs more gets a runtime
# allocation instead)
MI355X_MAX_SPLITK = 32
MI355X_SPLITK_CAP = 256 * 1024 * 1024

PROFILES = {
    "mi355x": MI355X_PROFILE,
    "cpu_generic": {"name": "cpu_generic", "backends": ["ref", "cpu", "simd"], "bnns": True,
                    "scratch_arena_max": 33554432, "activation_arena_max": 0},
    "cpu_generic_nobnns": {"name": "cpu_generic_nobnns", "backends": ["ref", "cpu", "simd"], "bnns": False,
                           "scratch_arena_max": 1 << 30, "activation_arena_max": 0},
    "cpu_ref": {"name": "cpu_ref", "backends": ["ref"], "scratch_arena_max": 1 << 30, "activation_arena_max": 0},
    # the reference's ARM profile (compiler/target/profiles/cpu_arm_neon.json):
    # Conv tokens int8, pointwise, depthwise, Winograd F(4,3), im2col; its
    # 32 MiB scratch limit (the 64 MiB activation limit is not checked by
    # this writer's planner, for any profile)
    "cpu_arm_neon": {"name": "cpu_arm_neon", "backends": ["ref", "cpu", "simd"], "bnns": False,
                     "conv_kinds": ["pointwise_1x1", "depthwise_direct", "winograd_f43"],
                     "scratch_arena_max": 33554432, "activation_arena_max": 0},
    # the two conv kinds the reference runtime keeps (spkv2_format.h:130-131,
    # kernels.c:75-77) but no reference profile selects: Winograd F(2,3) for
    # 3x3/s1/p1 and the 3x3/s2/p1 direct conv; packages carrying them must
    # still run unchanged
    "cpu_arm_neon_exp": {"name": "cpu_arm_neon_exp", "backends": ["ref", "cpu", "simd"], "bnns": False,
                         "conv_kinds": ["pointwise_1x1", "depthwise_direct", "winograd_3x3s1", "conv3x3s2_direct"],
                         "scratch_arena_max": 33554432, "activation_arena_max": 0},
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
    if kind in ("winograd_3x3s1", "winograd_f43"):
        # transformed input and output tiles (reference kernel_spec.py:244-263)
        side, alpha = (2, 16) if kind == "winograd_3x3s1" else (4, 36)
        tiles = ((y[2] + side - 1) // side) * ((y[3] + side - 1) // side)
        return _align(min(alpha * (x[1] + w[0]) * tiles * 4, SIMD_TILE_BYTES))
    if kind == "im2col_gemm":
        k = x[1] * w[2] * w[3]
        if backend == "simd":
            return _align(min(k * y[2] * y[3] * 4, 2 * 1024 * 1024))
        return _align(k * 4)
    return 0


def _align256(v: int) -> int:
    return (v + 255) // 256 * 256


def _mi355x_scratch(g: Graph, n: Node, kind: str) -> int:
    """Device workspace of an mi355x kind: the padded input copy the kernel
    gathers from (when some tap leaves the input) plus split-K partials."""
    if kind not in ("implicit_gemm_f32", "implicit_gemm_i8", "gemm_f32"):
        return 0
    if kind == "gemm_f32":
        if n.op_type != "Gemm":
            return 0
        a = g.tensors[n.inputs[0]].shape
        y = g.tensors[n.outputs[0]].shape
        rows = a[1] if int(n.attrs.get("transA", 0)) else a[0]
        return _align256(min(MI355X_MAX_SPLITK * int(y[-1]) * int(rows) * 4, MI355X_SPLITK_CAP))
    x, w, y = _conv_geometry(g, n)
    if int(n.attrs.get("group", 1)) != 1:
        return 0                                         # grouped: direct conv, no workspace
    N, C, H, W = (int(v) for v in x)
    M, KH, KW = int(w[0]), int(w[2]), int(w[3])
    OH, OW = int(y[2]), int(y[3])
    sh, sw = (int(v) for v in n.attrs.get("strides", [1, 1]))
    dh, dw = (int(v) for v in n.attrs.get("dilations", [1, 1]))
    pt, pl = (int(v) for v in list(n.attrs.get("pads", [0, 0, 0, 0]))[:2])
    hspan = (OH - 1) * sh + (KH - 1) * dh + 1
    wspan = (OW - 1) * sw + (KW - 1) * dw + 1
    Hp, Wp = max(H + pt, hspan), max(W + pl, wspan)
    partial = min(MI355X_MAX_SPLITK * M * N * OH * OW * 4, MI355X_SPLITK_CAP)
    if kind == "implicit_gemm_i8":
        cp = (C + 3) // 4 * 4 if dw == 1 else (C + 15) // 16 * 16
        return _align256(N * Hp * Wp * cp + 64) + partial
    padded = pt > 0 or pl > 0 or hspan - pt > H or wspan - pl > W
    return (_align256(N * C * Hp * Wp * 4) if padded else 0) + partial


def _mi355x_specs(g: Graph, n: Node, prof: dict) -> list[Spec]:
    """The op's applicable mi355x tokens, in the profile's order."""
    tokens = prof["ops"].get(n.op_type, [])
    if not tokens:
        raise ValueError(f"target profile does not support op: {n.op_type}")
    out = []
    for tok in tokens:
        if not tok.startswith("mi355x_"):
            raise ValueError(f"unknown mi355x profile token {tok}")
        kind = tok[len("mi355x_"):]
        dtype = "fp32"
        if n.op_type == "Conv":
            int8 = g.tensors[n.inputs[1]].dtype == "int8"
            if kind == "implicit_gemm_i8":
                if not int8:
                    continue
                dtype = "int8"
            elif int8:
                continue                                  # int8 weights need the int8 kernel
        out.append(Spec(0, n.id, kind, "mi355x", dtype, _mi355x_scratch(g, n, kind)))
    if not out:
        raise ValueError(f"no mi355x kernel applies to node {n.id} ({n.op_type})")
    return out


def _cpu_conv_kind(g: Graph, n: Node, prof: dict) -> str:
    """reference kernel_spec.py:146-224: the first conv kind of the profile's
    token list whose shape conditions the node meets (cpu_generic: bnns,
    pointwise, depthwise; cpu_arm_neon: pointwise, depthwise, Winograd
    F(4,3); the experimental list: F(2,3) and the 3x3/s2 direct conv),
    else im2col."""
    x, w, y = _conv_geometry(g, n)
    group = int(n.attrs.get("group", 1))
    strides = list(n.attrs.get("strides", [1, 1]))
    pads = list(n.attrs.get("pads", [0, 0, 0, 0]))
    dil = list(n.attrs.get("dilations", [1, 1]))
    k3 = w[2] == 3 and w[3] == 3 and dil == [1, 1] and group == 1 and pads == [1, 1, 1, 1]
    kinds = prof.get("conv_kinds", ["bnns_fp32", "pointwise_1x1", "depthwise_direct"])
    for kind in kinds:
        if kind == "bnns_fp32" and prof.get("bnns", True) and group == 1:
            return kind
        if (kind == "pointwise_1x1" and group == 1 and w[2] == 1 and w[3] == 1 and strides == [1, 1]
                and pads == [0, 0, 0, 0] and dil == [1, 1]):
            return kind
        if kind == "depthwise_direct" and group == x[1] and group == w[0] and w[2] == 3 and w[3] == 3 and dil == [1, 1]:
            return kind
        if kind == "winograd_f43" and k3 and strides == [1, 1]:
            oh, ow = y[2], y[3]
            tiles = ((oh + 3) // 4) * ((ow + 3) // 4)
            if (oh >= 8 and ow >= 8 and (x[1] >= 8 or w[0] >= 8) and tiles >= 4
                    and 36 * (x[1] + w[0]) * tiles * 4 <= SIMD_TILE_BYTES):
                return kind
        # the reference's x86 kernels of these two kinds take no residual
        # operand (optimized/conv/conv.c:1021-1048 pass none), so a conv with
        # a fused residual keeps im2col
        plain = len(n.inputs) < 4
        if kind == "winograd_3x3s1" and k3 and plain and strides == [1, 1] and y[2] == x[2] and y[3] == x[3]:
            return kind
        if kind == "conv3x3s2_direct" and k3 and plain and strides == [2, 2]:
            return kind
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
            chain = _mi355x_specs(g, n, prof)
            sel = add(chain[0])
            if len(chain) > 1:
                sel.fallback = add(chain[1]).id
        elif profile == "cpu_ref":
            sel = add(Spec(0, n.id, "reference", "ref"))
        else:
            ref = Spec(0, n.id, "reference", "ref")
            if n.op_type == "Conv":
                int8 = g.tensors[n.inputs[1]].dtype == "int8"
                if int8 and int(n.attrs.get("group", 1)) == 1:
                    sel = Spec(0, n.id, "int8_im2col_gemm", "simd", "int8")
                else:
                    sel = Spec(0, n.id, _cpu_conv_kind(g, n, prof), "simd")
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
    limit = prof["memory"]["scratch_arena_max"] if "memory" in prof else prof["scratch_arena_max"]
    if scratch > limit:
        raise MemoryError(f"scratch arena {scratch} exceeds profile limit {limit}")
    return specs, by_node, scratch
