"""INT8 quantization of a fused graph, with the reference's rules.

Weights (reference compiler/quantization/quantize_weights.py:24-83): every
group-1 Conv weight becomes int8 per output channel,
    s[c] = max(max|W[c]|, 1e-8) / 127            (float32)
    Wq[c] = clip(round_half_even(W[c] / s[c]), -128, 127).
Activations (reference calibrate.py:74-149): each Conv input gets a
per-tensor symmetric scale max|x| / 127 over the calibration samples (1.0
when all-zero), zero point 0.  The reference measures max|x| with
onnxruntime; here a float32 forward pass of the same fused graph (torch on
the host CPU) does it, and the scales are stored in the package, which is
all the runtime consumes.
"""

from __future__ import annotations

import numpy as np

from .graph import Graph
from .writer import QuantParam


def quantize_conv_weights(g: Graph) -> list[QuantParam]:
    params: list[QuantParam] = []
    done: set[int] = set()
    for n in g.nodes:
        if n.op_type != "Conv" or int(n.attrs.get("group", 1)) != 1:
            continue
        tid = n.inputs[1]
        t = g.tensors[tid]
        if tid in done or t.dtype != "fp32":
            continue
        w = t.data.astype(np.float32).reshape(t.shape[0], -1)
        cmax = np.maximum(np.max(np.abs(w), axis=1), np.float32(1e-8)).astype(np.float32)
        scales = (cmax / np.float32(127.0)).astype(np.float32)
        q = np.clip(np.round(w / scales[:, None]), -128, 127).astype(np.int8)
        t.data = q.reshape(t.shape)
        t.dtype = "int8"
        params.append(QuantParam(tid, "per_channel", 0, [float(s) for s in scales], [0] * len(scales)))
        done.add(tid)
    return params


def forward_fp32(g: Graph, inputs: list[np.ndarray], want: set[int]) -> dict[int, np.ndarray]:
    """float32 forward of a fused graph on the host (torch CPU), returning
    the tensors listed in `want`."""
    import torch
    import torch.nn.functional as F

    vals: dict[int, torch.Tensor] = {}
    for tid, x in zip(g.inputs, inputs):
        vals[tid] = torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32))
    for t in g.tensors:
        if t.role == "weight":
            vals[t.id] = torch.from_numpy(np.ascontiguousarray(t.data).astype(np.float32))

    def act(v, a):
        if a == "Relu":
            return torch.relu(v)
        if a == "Silu":
            return v * torch.sigmoid(v)
        return v

    out: dict[int, np.ndarray] = {}
    with torch.no_grad():
        for n in g.nodes:
            a = n.attrs
            x = vals[n.inputs[0]]
            if n.op_type == "Conv":
                p = a.get("pads", [0, 0, 0, 0])
                xp = F.pad(x, (p[1], p[3], p[0], p[2]))
                y = F.conv2d(xp, vals[n.inputs[1]], vals[n.inputs[2]] if len(n.inputs) > 2 else None,
                             stride=a.get("strides", [1, 1]), dilation=a.get("dilations", [1, 1]),
                             groups=a.get("group", 1))
                if len(n.inputs) > 3:
                    y = y + vals[n.inputs[3]]
                y = act(y, a.get("fused_activation"))
            elif n.op_type == "MaxPool":
                p = a["pads"]
                y = F.max_pool2d(F.pad(x, (p[1], p[3], p[0], p[2]), value=float("-inf")), a["kernel_shape"],
                                 a["strides"])
            elif n.op_type == "Add":
                y = act(x + vals[n.inputs[1]], a.get("fused_activation"))
            elif n.op_type == "Relu":
                y = torch.relu(x)
            elif n.op_type == "ReduceMean":
                y = x.mean(dim=tuple(a["axes"]), keepdim=bool(a.get("keepdims", 1)))
            elif n.op_type in ("Flatten", "Reshape"):
                y = x.reshape(g.shape(n.outputs[0]))
            elif n.op_type == "Gemm":
                w = vals[n.inputs[1]]
                xa = x.T if a.get("transA") else x
                y = a.get("alpha", 1.0) * (xa @ (w.T if a.get("transB") else w))
                if len(n.inputs) > 2:
                    y = y + vals[n.inputs[2]]
            elif n.op_type == "Softmax":
                y = torch.softmax(x, dim=a.get("axis", -1))
            elif n.op_type == "GlobalAveragePool":
                y = x.mean(dim=(2, 3), keepdim=True)
            else:
                raise NotImplementedError(n.op_type)
            vals[n.outputs[0]] = y
            if n.outputs[0] in want:
                out[n.outputs[0]] = y.numpy()
        for tid in want:
            if tid not in out and tid in vals:
                out[tid] = vals[tid].numpy()
    return out


def calibrate_activation_scales(g: Graph, samples: list) -> list[QuantParam]:
    """Per-tensor scale of every Conv input over the calibration samples
    (each sample: one input array, or a list with one array per graph input)."""
    conv_inputs = []
    for n in g.nodes:
        if n.op_type == "Conv" and n.inputs[0] not in conv_inputs:
            conv_inputs.append(n.inputs[0])
    max_abs: dict[int, float] = {}
    for s in samples:
        vals = forward_fp32(g, s if isinstance(s, (list, tuple)) else [s], set(conv_inputs))
        for tid in conv_inputs:
            m = float(np.max(np.abs(vals[tid])))
            max_abs[tid] = max(max_abs.get(tid, 0.0), m)
    params = []
    for tid in conv_inputs:
        m = max_abs[tid]
        scale = m / 127.0 if m > 0 else 1.0  # float64 quotient, stored as float32
        params.append(QuantParam(tid, "per_tensor", 0, [scale], [0]))
    return params


def quantize_graph(g: Graph, samples: list[np.ndarray]) -> list[QuantParam]:
    """Calibrate on the fp32 graph, then quantize its conv weights."""
    act = calibrate_activation_scales(g, samples)
    wq = quantize_conv_weights(g)
    return wq + act


# ----------------------------------------------------------------------------
# INT8 with int8 tensors between nodes (the benchmark's INT8 configuration).
#
# The reference quantizes activations symmetrically with zero point 0 and
# keeps fp32 tensors between nodes (calibrate.py:16, conv_int8.c:86-119).
# This mode is the configuration's own: per-channel symmetric int8 weights
# (the rule above), per-tensor asymmetric activation scales and zero points
# from min/max over the calibration samples, and the tensors between the
# quantized nodes stored as int8 (package dtype int8, role activation).  A
# Conv in this mode accumulates in int32 and requantizes in fixed point with
# round-half-away into its int8 output; MaxPool passes int8 through (its
# output shares its input's scale and zero point); ReduceMean over H, W (or
# GlobalAveragePool) dequantizes to fp32.


def asymmetric_params(lo: float, hi: float) -> tuple[float, int]:
    """(scale, zero point) of a per-tensor asymmetric int8 range: the range
    widened to hold 0, s = (hi - lo) / 255 as float32 (1.0 for an empty
    range), z = round_half_away(-128 - lo / s) clamped to [-128, 127]."""
    lo, hi = min(float(lo), 0.0), max(float(hi), 0.0)
    s = float(np.float32((hi - lo) / 255.0)) if hi > lo else 1.0
    v = -128.0 - lo / s
    z = int(np.floor(v + 0.5)) if v >= 0 else -int(np.floor(-v + 0.5))
    return s, max(-128, min(127, z))


def _int8_capable_reader(g: Graph, n, idx: int) -> bool:
    if n.op_type == "Conv":
        w = g.tensors[n.inputs[1]]
        return idx in (0, 3) and int(n.attrs.get("group", 1)) == 1 and len(w.shape) == 4
    if n.op_type == "MaxPool":
        return idx == 0
    if n.op_type == "ReduceMean":
        return idx == 0 and len(g.shape(n.inputs[0])) == 4 and sorted(int(a) % 4 for a in n.attrs.get("axes", [])) == [2, 3]
    return n.op_type == "GlobalAveragePool" and idx == 0


def int8_tensor_plan(g: Graph) -> tuple[set[int], list]:
    """The tensors the mode stores as int8 and the Convs it runs: the output
    of a group-1 Conv without SiLU, or of a MaxPool, becomes int8 when it is
    not a graph output and every reader takes int8 (a group-1 Conv as input
    or residual, a MaxPool, a spatial mean); a Conv runs in the mode only when its output is
    int8, so its int8 inputs and residual must be too, and a MaxPool keeps
    int8 only with int8 on both sides.  Iterated to a fixed point."""
    readers: dict[int, list] = {}
    for n in g.nodes:
        for i, t in enumerate(n.inputs):
            readers.setdefault(t, []).append((n, i))
    cand = set()
    for n in g.nodes:
        # the requantizing epilogue applies Relu as a clamp; a SiLU conv keeps
        # its fp32 output
        q8_conv = (n.op_type == "Conv" and int(n.attrs.get("group", 1)) == 1 and
                   n.attrs.get("fused_activation") in (None, "Relu"))
        if q8_conv or n.op_type == "MaxPool":
            t = n.outputs[0]
            if t not in g.outputs and readers.get(t) and all(_int8_capable_reader(g, r, i) for r, i in readers[t]):
                cand.add(t)
    changed = True
    while changed:
        changed = False
        for n in g.nodes:
            if n.op_type == "Conv" and int(n.attrs.get("group", 1)) == 1:
                out_q = n.outputs[0] in cand
                res = n.inputs[3] if len(n.inputs) > 3 else None
                if out_q and res is not None and res not in cand:
                    cand.discard(n.outputs[0])
                    changed = True
                    out_q = False
                if not out_q:
                    for t in (n.inputs[0], res):
                        if t is not None and t in cand:
                            cand.discard(t)
                            changed = True
            elif n.op_type == "MaxPool":
                i, o = n.inputs[0], n.outputs[0]
                if (i in cand) != (o in cand):
                    cand.discard(i)
                    cand.discard(o)
                    changed = True
    convs = [n for n in g.nodes if n.op_type == "Conv" and n.outputs[0] in cand]
    return cand, convs


def quantize_int8_activations(g: Graph, samples: list, calibrate_on: Graph | None = None) -> list[QuantParam]:
    """Turns a fused fp32 graph into the INT8 configuration's package form:
    calibrates min/max of every tensor the mode stores as int8 (and of the
    fp32 inputs its Convs quantize on load) on the samples with the fp32
    forward, quantizes those Convs' weights per channel, marks the int8
    tensors, and returns the quantization records (per-tensor scale and
    zero point; MaxPool outputs take their input's).  `calibrate_on` runs
    the samples through another graph of the same structure and weights
    (e.g. the batch-1 graph for a batch-64 package: tensor ids agree)."""
    cand, convs = int8_tensor_plan(g)
    if not convs:
        raise ValueError("no Conv of this graph can run with int8 tensors between nodes")
    fp32_in = {n.inputs[0] for n in convs if n.inputs[0] not in cand}
    readers_ref = {n.inputs[0] for n in g.nodes if n.op_type == "Conv" and n not in convs}
    if fp32_in & readers_ref:
        raise ValueError("an fp32 tensor feeds Convs of both INT8 modes (one quantization record per tensor)")
    want = cand | fp32_in
    lo: dict[int, float] = {}
    hi: dict[int, float] = {}
    for smp in samples:
        vals = forward_fp32(calibrate_on or g, smp if isinstance(smp, (list, tuple)) else [smp], want)
        for t in want:
            v = vals[t]
            lo[t] = min(lo.get(t, np.inf), float(np.min(v)))
            hi[t] = max(hi.get(t, -np.inf), float(np.max(v)))
    params: dict[int, tuple[float, int]] = {t: asymmetric_params(lo[t], hi[t]) for t in want}
    for n in g.nodes:  # topological order: a pool's input is settled first
        if n.op_type == "MaxPool" and n.outputs[0] in cand:
            params[n.outputs[0]] = params[n.inputs[0]]
    out: list[QuantParam] = []
    done: set[int] = set()
    for n in convs:
        tid = n.inputs[1]
        t = g.tensors[tid]
        if tid in done or t.dtype != "fp32":
            continue
        w = t.data.astype(np.float32).reshape(t.shape[0], -1)
        cmax = np.maximum(np.max(np.abs(w), axis=1), np.float32(1e-8)).astype(np.float32)
        scales = (cmax / np.float32(127.0)).astype(np.float32)
        t.data = np.clip(np.round(w / scales[:, None]), -128, 127).astype(np.int8).reshape(t.shape)
        t.dtype = "int8"
        out.append(QuantParam(tid, "per_channel", 0, [float(s) for s in scales], [0] * len(scales)))
        done.add(tid)
    for t in sorted(want):
        s, z = params[t]
        out.append(QuantParam(t, "per_tensor", 0, [s], [z]))
        if t in cand:
            g.tensors[t].dtype = "int8"
    return out
