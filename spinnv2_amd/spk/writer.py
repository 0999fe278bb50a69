"""SPK v0.3 package writer.

Produces the section set, order and alignment the reference writer produces
(compiler/packager/spk_writer.py:109-199): metadata JSON, target profile JSON,
tensor / node / attr tables, 4096-aligned weights (each tensor 16-aligned),
memory plan, kernel specs, optional quantization, string table, and the
FNV-1a checksum over everything before the checksum section.
"""

from __future__ import annotations

import json
import math
from dataclasses import dataclass, field
from pathlib import Path

import numpy as np

from . import format as F
from .graph import Graph, Node
from .kernel_spec import PROFILES, select_kernel_specs
from .planner import plan_memory


@dataclass
class QuantParam:
    tensor_id: int
    scheme: str  # per_tensor | per_channel
    quant_axis: int
    scales: list[float]
    zero_points: list[int] = field(default_factory=list)


def _align(v: int, a: int) -> int:
    return (v + a - 1) // a * a


def _ints(v, n: int, default: int) -> list[int]:
    return ([int(x) for x in v] + [default] * n)[:n]


def attr_bytes(n: Node) -> bytes:
    """One 124-byte attr record (layout of reference spk_writer.py:236-293)."""
    a = n.attrs
    extra: list[int] = []
    if n.op_type == "Transpose":
        extra = [int(v) for v in a.get("perm", [])]
    elif n.op_type in ("ReduceMean", "ReduceMax") and "axes" in a:
        extra = [int(v) for v in a["axes"]]
    pads = _ints(a.get("pads", [0, 0, 0, 0]), 4, 0)
    return F.ATTR.pack(
        F.OP[n.op_type], int(a.get("axis", 1)), int(a.get("group", 1)), F.ACTIVATION[a.get("fused_activation")],
        *pads, *_ints(a.get("strides", [1, 1]), 2, 1), *_ints(a.get("kernel_shape", [1, 1]), 2, 1),
        *_ints(a.get("dilations", [1, 1]), 2, 1), int(a.get("transA", 0)), int(a.get("transB", 0)),
        float(a.get("alpha", 1.0)), float(a.get("beta", 1.0)), len(extra), int(a.get("keepdims", 1)),
        *(extra + [0] * 8)[:8], int(a.get("largest", 1)), int(a.get("sorted", 1)), int(a.get("to", 1)),
    )


def _quant_section(params: list[QuantParam]) -> bytes:
    records_size = len(params) * F.QUANT_PARAM.size
    data = bytearray()
    offsets = []
    for q in params:
        offsets.append(records_size + len(data))
        data += np.asarray(q.scales, dtype="<f4").tobytes()
        zps = q.zero_points or [0] * len(q.scales)
        data += np.asarray(zps, dtype="<i4").tobytes()
    recs = bytearray()
    for q, off in zip(params, offsets):
        recs += F.QUANT_PARAM.pack(q.tensor_id, F.QUANT_SCHEME[q.scheme], q.quant_axis, len(q.scales), off)
    return bytes(recs + data)


@dataclass
class Protection:
    """One protection-plan entry (reference compiler/reliability/
    protection_plan.py:15-24): `mode` is "range_guard_rerun" (bounds on the
    node's single fp32 output) or "dmr_compare_rerun" (run twice, compare
    bytes, rerun on mismatch; scratch for two copies of the output)."""
    node_id: int
    mode: str
    lower_bound: float = -math.inf
    upper_bound: float = math.inf


PROTECTION_MODES = {"none": 0, "range_guard_rerun": 1, "dmr_compare_rerun": 2}


def _protection_section(g: Graph, entries: list[Protection], scratch_offset: int) -> tuple[bytes, int]:
    """Records in the reference's encoding (protection_plan.py:65-81):
    infinite bounds as +-FLT_MAX, the DMR scratch right after the kernels'
    scratch arena.  Returns the records and the extra scratch bytes."""
    out = bytearray()
    extra = 0
    seen = set()
    for e in entries:
        n = g.nodes[e.node_id]
        if e.node_id in seen or len(n.outputs) != 1 or g.tensors[n.outputs[0]].dtype != "fp32":
            raise ValueError(f"node {e.node_id} cannot be protected")
        if e.mode == "range_guard_rerun" and e.lower_bound > e.upper_bound:
            raise ValueError(f"invalid range for node {e.node_id}")
        seen.add(e.node_id)
        lower = e.lower_bound if math.isfinite(e.lower_bound) else -3.4028235e38
        upper = e.upper_bound if math.isfinite(e.upper_bound) else 3.4028235e38
        dmr = e.mode == "dmr_compare_rerun"
        if dmr:
            extra = max(extra, 2 * g.tensors[n.outputs[0]].size_bytes)
        out += F.PROTECTION.pack(e.node_id, n.outputs[0], PROTECTION_MODES[e.mode], 0, lower, upper,
                                 scratch_offset if dmr else 0)
    return bytes(out), extra


def write_spk(g: Graph, profile: str = "mi355x", *, quant_params: list[QuantParam] | None = None,
              path: str | Path | None = None, external_inputs: bool = False,
              external_outputs: bool = False, protection: list[Protection] | None = None) -> bytes:
    g.relink()
    bad = sorted({n.op_type for n in g.nodes if n.op_type not in F.OP})
    if bad:
        raise ValueError(f"graph still contains ops the runtime does not know: {bad}")
    specs, by_node, scratch = select_kernel_specs(g, profile)
    plan = plan_memory(g, external_inputs=external_inputs, external_outputs=external_outputs)

    # strings
    strings = bytearray(b"\x00")
    name_off: dict[str, int] = {"": 0}
    for t in g.tensors:
        if t.name not in name_off:
            name_off[t.name] = len(strings)
            strings += t.name.encode() + b"\x00"

    # weights
    weights = bytearray()
    w_off: dict[int, int] = {}
    for t in g.tensors:
        if t.role != "weight":
            continue
        weights += b"\x00" * (_align(len(weights), 16) - len(weights))
        w_off[t.id] = len(weights)
        arr = t.data.astype({"int8": np.int8, "fp16": "<f2"}.get(t.dtype, "<f4"), copy=False)
        weights += np.ascontiguousarray(arr).tobytes()

    # attrs
    attrs = bytearray()
    a_off: dict[int, tuple[int, int]] = {}
    for n in g.nodes:
        attrs += b"\x00" * (_align(len(attrs), 4) - len(attrs))
        blob = attr_bytes(n)
        a_off[n.id] = (len(attrs), len(blob))
        attrs += blob

    tensor_tab = bytearray()
    for t in g.tensors:
        e = plan.entries[t.id]
        shape = (list(t.shape) + [1] * 8)[:8]
        tensor_tab += F.TENSOR.pack(t.id, F.DTYPE[t.dtype], F.ROLE[t.role], len(t.shape),
                                    F.MEMORY_CLASS[e.memory_class], *shape, t.size_bytes,
                                    w_off.get(t.id, e.offset), name_off[t.name], 0)
    node_tab = bytearray()
    for n in g.nodes:
        ins = (n.inputs + [0] * 8)[:8]
        outs = (n.outputs + [0] * 4)[:4]
        s = by_node[n.id]
        node_tab += F.NODE.pack(n.id, F.OP[n.op_type], 0, len(n.inputs), len(n.outputs), *ins, *outs,
                                a_off[n.id][0], a_off[n.id][1], s.id, s.scratch_bytes)
    plan_tab = bytearray()
    for t in g.tensors:
        e = plan.entries[t.id]
        plan_tab += F.MEMORY_PLAN.pack(t.id, F.MEMORY_CLASS[e.memory_class], 16, 0, e.offset, e.size,
                                       e.first_use if e.first_use >= 0 else 0xFFFFFFFF,
                                       e.last_use if e.last_use >= 0 else 0xFFFFFFFF)
    spec_tab = bytearray()
    for s in specs:
        feat = {"fp32": 1, "int8": 2, "fp16": 4}[s.dtype]
        spec_tab += F.KERNEL_SPEC.pack(s.id, s.node_id, F.KIND[s.kind], F.BACKEND[s.backend], F.DTYPE[s.dtype], 1, 1,
                                       0, 0, s.scratch_bytes, s.fallback, feat)

    meta = json.dumps({"model_name": g.model_name, "sir_version": "0.1", "inputs": g.inputs,
                       "outputs": g.outputs}, sort_keys=True).encode()
    prof_json = json.dumps(PROFILES[profile], sort_keys=True).encode()
    sections: list[tuple[int, bytes, int]] = [
        (F.SECTION_METADATA, meta, 1),
        (F.SECTION_TARGET_PROFILE, prof_json, 1),
        (F.SECTION_TENSOR_TABLE, bytes(tensor_tab), 4),
        (F.SECTION_NODE_TABLE, bytes(node_tab), 4),
        (F.SECTION_ATTRIBUTES, bytes(attrs), 4),
        (F.SECTION_WEIGHTS, bytes(weights), 4096),
        (F.SECTION_MEMORY_PLAN, bytes(plan_tab), 4),
        (F.SECTION_KERNEL_SPEC, bytes(spec_tab), 4),
    ]
    if quant_params:
        sections.append((F.SECTION_QUANTIZATION, _quant_section(quant_params), 4))
    if protection:
        prot, extra_scratch = _protection_section(g, protection, scratch)
        sections.append((F.SECTION_PROTECTION_PLAN, prot, 8))
        scratch += extra_scratch
    sections.append((F.SECTION_STRING_TABLE, bytes(strings), 1))
    sections.append((F.SECTION_CHECKSUM, b"\x00" * 4, 4))

    offset = F.HEADER.size + len(sections) * F.SECTION.size
    directory = bytearray()
    payload = bytearray()
    checksum_at = 0
    for kind, data, align in sections:
        aligned = _align(offset, align)
        payload += b"\x00" * (aligned - offset)
        offset = aligned
        if kind == F.SECTION_CHECKSUM:
            checksum_at = offset
        directory += F.SECTION.pack(kind, 0, offset, len(data), align, 0)
        payload += data
        offset += len(data)
    header = F.HEADER.pack(
        F.MAGIC, F.VERSION_MAJOR, F.VERSION_MINOR, 0, F.HEADER.size, len(sections), 0, len(g.tensors), len(g.nodes),
        len(g.inputs), len(g.outputs), sum(t.size_bytes for t in g.tensors if t.role == "weight"), plan.arena_bytes,
        scratch, F.fnv1a32(prof_json), 1)
    pkg = bytearray(header + directory + payload)
    pkg[checksum_at:checksum_at + 4] = F.fnv1a32(pkg[:checksum_at]).to_bytes(4, "little")
    out = bytes(pkg)
    if path is not None:
        Path(path).write_bytes(out)
    return out
