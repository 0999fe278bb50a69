"""Static activation-arena planning.

Rules follow the reference planner (compiler/planner/memory_plan.py):
  - lifetime of a tensor = [producer node, last consumer]; graph outputs live
    to the end; inputs start at node 0;
  - 16-byte aligned best-fit placement in order of first use, freed blocks
    coalesced;
  - in-place aliases: Reshape / Flatten / Unsqueeze / Cast outputs, and Relu
    outputs whose input has a single consumer, share their input's offset
    (memory_plan.py:15-16, 269-297);
  - Concat sub-region aliases: when everything before the axis has extent 1,
    each input is placed inside the Concat output at axis_offset*inner*4
    bytes (memory_plan.py:300-380).
The offsets become each tensor record's data_offset, which the runtime maps
1:1 onto its device arena.
"""

from __future__ import annotations

from dataclasses import dataclass

from .graph import Graph

ALIGN = 16
SHAPE_ONLY = {"Reshape", "Flatten", "Unsqueeze", "Cast"}
ELEMENTWISE_INPLACE = {"Relu"}


def _align(v: int, a: int = ALIGN) -> int:
    return (v + a - 1) // a * a


@dataclass
class PlanEntry:
    tensor_id: int
    offset: int
    size: int
    first_use: int
    last_use: int
    memory_class: str


@dataclass
class MemoryPlan:
    entries: dict[int, PlanEntry]
    arena_bytes: int
    naive_bytes: int


def _allocated(t) -> bool:
    return t.role not in ("weight", "constant") and t.size_bytes > 0


def _memory_class(t, external_inputs: bool, external_outputs: bool) -> str:
    if t.role in ("weight", "constant"):
        return "WEIGHT"
    if t.role == "input":
        return "EXTERNAL" if external_inputs else "INPUT"
    if t.role == "output":
        return "EXTERNAL" if external_outputs else "OUTPUT"
    return "ACTIVATION_ARENA"


def plan_memory(g: Graph, *, external_inputs: bool = False, external_outputs: bool = False) -> MemoryPlan:
    g.relink()
    end = len(g.nodes) + 1
    life: dict[int, list[int]] = {}
    outs = set(g.outputs)
    for t in g.tensors:
        if t.role == "weight":
            life[t.id] = [-1, end]
            continue
        first = 0 if t.producer is None else t.producer
        last = end if t.id in outs else (max(t.consumers) if t.consumers else first)
        life[t.id] = [first, last]

    def placed(t) -> bool:
        if not _allocated(t):
            return False
        if t.role == "input" and external_inputs:
            return False
        if t.role == "output" and external_outputs:
            return False
        return True

    # in-place aliases
    alias: dict[int, int] = {}
    ins = set(g.inputs)
    for n in g.nodes:
        shape_only = n.op_type in SHAPE_ONLY
        eltwise = n.op_type in ELEMENTWISE_INPLACE
        if not (shape_only or eltwise) or not n.inputs or not n.outputs:
            continue
        src, dst = n.inputs[0], n.outputs[0]
        ts, td = g.tensors[src], g.tensors[dst]
        if ts.size_bytes != td.size_bytes or not placed(ts) or not placed(td):
            continue
        if dst in outs and src in ins:
            continue
        if eltwise and len(ts.consumers) > 1:
            continue
        root = alias.get(src, src)
        if eltwise and root in ins:
            continue
        alias[dst] = root

    # Concat sub-region aliases
    concat: dict[int, tuple[int, int]] = {}
    used: set[int] = set()
    for n in g.nodes:
        if n.op_type != "Concat" or len(n.inputs) < 2:
            continue
        out = g.tensors[n.outputs[0]]
        if not placed(out) or n.outputs[0] in alias:
            continue
        axis = int(n.attrs.get("axis", 0)) % len(out.shape)
        outer = 1
        for d in out.shape[:axis]:
            outer *= d
        if outer != 1:
            continue
        inner = 1
        for d in out.shape[axis + 1:]:
            inner *= d
        offs, ok, ax = [], True, 0
        for tid in n.inputs:
            t = g.tensors[tid]
            if not placed(t) or tid in ins or tid in used or tid in alias or tid in concat \
                    or any(v == tid for v in alias.values()):
                ok = False
                break
            byte_off = ax * inner * 4
            if byte_off % ALIGN:
                ok = False
                break
            offs.append((tid, byte_off))
            ax += t.shape[axis]
        if ok and len(set(n.inputs)) == len(n.inputs):
            for tid, off in offs:
                concat[tid] = (n.outputs[0], off)
                used.add(tid)

    for a, src in alias.items():
        life[src] = [min(life[src][0], life[a][0]), max(life[src][1], life[a][1])]
    for a, (parent, _) in concat.items():
        life[parent] = [min(life[parent][0], life[a][0]), max(life[parent][1], life[a][1])]

    roots = [t for t in g.tensors if placed(t) and t.id not in alias and t.id not in concat]
    naive = sum(_align(t.size_bytes) for t in roots)
    free: list[list[int]] = []  # [offset, size], sorted and coalesced
    active: list[tuple[int, int, int]] = []
    peak = 0
    offset: dict[int, int] = {}

    def release(off: int, size: int) -> None:
        free.append([off, size])
        free.sort()
        merged: list[list[int]] = []
        for b in free:
            if merged and merged[-1][0] + merged[-1][1] == b[0]:
                merged[-1][1] += b[1]
            else:
                merged.append(b)
        free[:] = merged

    for t in sorted(roots, key=lambda t: (life[t.id][0], t.id)):
        first = life[t.id][0]
        keep = []
        for tid, off, size in active:
            if life[tid][1] < first:
                release(off, size)
            else:
                keep.append((tid, off, size))
        active = keep
        size = _align(t.size_bytes)
        best = None
        for i, (off, bsize) in enumerate(free):
            if bsize >= size and (best is None or bsize < free[best][1]):
                best = i
        if best is None:
            off = peak
            peak += size
        else:
            off, bsize = free.pop(best)
            if bsize > size:
                release(off + size, bsize - size)
        offset[t.id] = off
        active.append((t.id, off, size))

    entries: dict[int, PlanEntry] = {}
    for t in g.tensors:
        if t.id in offset:
            off = offset[t.id]
        elif t.id in alias:
            off = offset[alias[t.id]]
        elif t.id in concat:
            parent, boff = concat[t.id]
            root = alias.get(parent, parent)
            off = offset[root] + boff
        else:
            off = 0
        first, last = life.get(t.id, [-1, -1])
        entries[t.id] = PlanEntry(t.id, off, t.size_bytes, first, last,
                                  _memory_class(t, external_inputs, external_outputs))
    return MemoryPlan(entries, peak, naive)
