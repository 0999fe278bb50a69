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
