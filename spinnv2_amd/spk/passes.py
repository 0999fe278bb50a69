"""Graph fusions that decide what the node kernels must fuse.

Each pass follows the matching reference pass (compiler/passes/transforms.py)
and they run in the reference's default order (compiler/passes/manager.py:39-50):
BN folding, Conv+Relu, Conv+SiLU, Add+Relu, Conv+Add.
"""

from __future__ import annotations

import numpy as np

from .graph import Graph


def _single_consumer(g: Graph, tid: int, consumer: int) -> bool:
    others = [c for c in g.tensors[tid].consumers if c != consumer]
    return not others and tid not in g.outputs


def _remove(g: Graph, drop: set[int]) -> None:
    g.nodes = [n for n in g.nodes if n.id not in drop]
    g.compact()


def fold_batchnorm(g: Graph) -> int:
    """Conv -> BatchNormalization  =>  Conv with
    w' = w * gamma / sqrt(var + eps),  b' = gamma * (b - mean) / sqrt(var + eps) + beta
    computed in float32 (reference transforms.py:63-116)."""
    g.relink()
    drop: set[int] = set()
    for bn in list(g.nodes):
        if bn.op_type != "BatchNormalization":
            continue
        conv_id = g.tensors[bn.inputs[0]].producer
        if conv_id is None or g.nodes[conv_id].op_type != "Conv":
            continue
        conv = g.nodes[conv_id]
        if not _single_consumer(g, bn.inputs[0], bn.id):
            continue
        gamma, beta, mean, var = (g.tensors[t].data.astype(np.float32) for t in bn.inputs[1:5])
        eps = np.float32(bn.attrs.get("epsilon", 1e-5))
        w_t = g.tensors[conv.inputs[1]]
        oc = w_t.shape[0]
        factor = gamma.reshape(oc) / np.sqrt(var.reshape(oc) + eps)
        w_t.data = (w_t.data * factor.reshape(oc, 1, 1, 1)).astype(np.float32)
        if len(conv.inputs) >= 3:
            b_t = g.tensors[conv.inputs[2]]
            old_b = b_t.data.reshape(oc)
        else:
            old_b = np.zeros((oc,), np.float32)
            b_id = g.weight(f"{w_t.name}_bn_bias", old_b)
            conv.inputs.append(b_id)
            b_t = g.tensors[b_id]
        b_t.data = (factor * (old_b - mean.reshape(oc)) + beta.reshape(oc)).astype(np.float32)
        conv.outputs[0] = bn.outputs[0]
        drop.add(bn.id)
    if drop:
        _remove(g, drop)
    return len(drop)


def fuse_conv_relu(g: Graph) -> int:
    """Conv -> Relu => Conv(fused_activation=Relu) (reference transforms.py:119-143)."""
    g.relink()
    drop: set[int] = set()
    for relu in list(g.nodes):
        if relu.op_type != "Relu":
            continue
        pid = g.tensors[relu.inputs[0]].producer
        if pid is None or g.nodes[pid].op_type != "Conv" or pid in drop:
            continue
        conv = g.nodes[pid]
        if conv.attrs.get("fused_activation") or not _single_consumer(g, relu.inputs[0], relu.id):
            continue
        conv.attrs["fused_activation"] = "Relu"
        conv.outputs[0] = relu.outputs[0]
        drop.add(relu.id)
    if drop:
        _remove(g, drop)
    return len(drop)


def fuse_conv_silu(g: Graph) -> int:
    """Conv -> {Sigmoid, Mul(conv, sigmoid)} => Conv(fused_activation=Silu)
    (reference transforms.py:146-178)."""
    g.relink()
    drop: set[int] = set()
    for conv in list(g.nodes):
        if conv.op_type != "Conv" or conv.attrs.get("fused_activation"):
            continue
        out = conv.outputs[0]
        cons = [g.nodes[c] for c in g.tensors[out].consumers]
        if len(cons) != 2 or out in g.outputs:
            continue
        sig = next((n for n in cons if n.op_type == "Sigmoid"), None)
        mul = next((n for n in cons if n.op_type == "Mul"), None)
        if sig is None or mul is None:
            continue
        if not _single_consumer(g, sig.outputs[0], mul.id) or set(mul.inputs) != {out, sig.outputs[0]}:
            continue
        conv.attrs["fused_activation"] = "Silu"
        conv.outputs[0] = mul.outputs[0]
        drop.update({sig.id, mul.id})
    if drop:
        _remove(g, drop)
    return len(drop) // 2


def fuse_add_relu(g: Graph) -> int:
    """Add -> Relu => Add(fused_activation=Relu) (reference transforms.py:181-206)."""
    g.relink()
    drop: set[int] = set()
    for relu in list(g.nodes):
        if relu.op_type != "Relu":
            continue
        pid = g.tensors[relu.inputs[0]].producer
        if pid is None or g.nodes[pid].op_type != "Add" or pid in drop:
            continue
        add = g.nodes[pid]
        if add.attrs.get("fused_activation") or not _single_consumer(g, relu.inputs[0], relu.id):
            continue
        add.attrs["fused_activation"] = "Relu"
        add.outputs[0] = relu.outputs[0]
        drop.add(relu.id)
    if drop:
        _remove(g, drop)
    return len(drop)


def fuse_conv_add(g: Graph) -> int:
    """Conv -> Add(conv, r) => Conv(x, w, b, r) with the Add's activation,
    applied after the residual (reference transforms.py:209-256).  A conv that
    already carries an activation is not fused; a missing bias becomes zeros."""
    g.relink()
    drop: set[int] = set()
    for add in list(g.nodes):
        if add.op_type != "Add" or len(add.inputs) != 2:
            continue
        for side in (0, 1):
            conv_out, res = add.inputs[side], add.inputs[1 - side]
            pid = g.tensors[conv_out].producer
            if pid is None or g.nodes[pid].op_type != "Conv" or pid in drop:
                continue
            conv = g.nodes[pid]
            if conv.attrs.get("fused_activation") or not _single_consumer(g, conv_out, add.id):
                continue
            if g.shape(conv_out) != g.shape(add.outputs[0]) or g.shape(res) != g.shape(add.outputs[0]):
                continue
            if len(conv.inputs) < 3:
                oc = g.tensors[conv.inputs[1]].shape[0]
                conv.inputs.append(g.weight(f"{g.tensors[conv.inputs[1]].name}_zero_bias", np.zeros(oc, np.float32)))
            conv.inputs.append(res)
            if add.attrs.get("fused_activation"):
                conv.attrs["fused_activation"] = add.attrs["fused_activation"]
            conv.outputs[0] = add.outputs[0]
            drop.add(add.id)
            break
    if drop:
        # the residual producer may now come after the conv: restore topological order
        g.nodes = [n for n in g.nodes if n.id not in drop]
        _toposort(g)
        g.compact()
    return len(drop)


def _toposort(g: Graph) -> None:
    produced = {t for t in g.inputs} | {t.id for t in g.tensors if t.role == "weight"}
    pending = list(g.nodes)
    ordered = []
    while pending:
        progressed = False
        for n in list(pending):
            if all(t in produced for t in n.inputs):
                ordered.append(n)
                produced.update(n.outputs)
                pending.remove(n)
                progressed = True
        if not progressed:
            raise ValueError("graph has a cycle")
    g.nodes = ordered


DEFAULT_PIPELINE = [fold_batchnorm, fuse_conv_relu, fuse_conv_silu, fuse_add_relu, fuse_conv_add]


def convert_weights_fp16(g: Graph) -> int:
    """Stores every fp32 weight of rank >= 2 as IEEE half (round to nearest
    even), as the reference's --fp16-weights pass does
    (compiler/passes/convert_fp16.py:11-25); biases and scalars stay fp32.
    The runtime widens them back to fp32 once at load.  Returns the number
    of tensors converted."""
    count = 0
    for t in g.tensors:
        if t.role == "weight" and t.dtype == "fp32" and t.data is not None and len(t.shape) >= 2:
            t.data = np.asarray(t.data, dtype=np.float32).astype(np.float16)
            t.dtype = "fp16"
            count += 1
    return count


def run_default_pipeline(g: Graph, *, conv_add: bool = True) -> dict[str, int]:
    stats = {}
    for p in DEFAULT_PIPELINE:
        if p is fuse_conv_add and not conv_add:
            continue
        stats[p.__name__] = p(g)
    return stats
