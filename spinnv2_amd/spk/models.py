"""Seeded generators for the benchmark and parity graphs.

Each builder emits the ONNX-level graph (Conv, BatchNormalization, Relu, Add,
...) with weights drawn from numpy's PCG64 generator, then runs the fusion
pipeline, so the packaged graph is what the reference compiler would produce
from the same model (BN folded, Conv+Relu, Add+Relu, Conv+Add).

Distributions: conv / fc weights He-normal
N(0, sqrt(2 / fan_in)); biases N(0, 0.01); BN gamma ~ U(0.5, 1.5),
beta, mean ~ N(0, 0.1), var ~ U(0.5, 1.5), eps 1e-5.
"""

from __future__ import annotations

import numpy as np

from .graph import Graph
from .passes import run_default_pipeline

DEFAULT_SEED = 42


class Params:
    def __init__(self, seed: int) -> None:
        self.rng = np.random.Generator(np.random.PCG64(seed))

    def he(self, shape) -> np.ndarray:
        fan_in = int(np.prod(shape[1:]))
        return (self.rng.standard_normal(shape, dtype=np.float64) * np.sqrt(2.0 / fan_in)).astype(np.float32)

    def normal(self, shape, std: float) -> np.ndarray:
        return (self.rng.standard_normal(shape, dtype=np.float64) * std).astype(np.float32)

    def uniform(self, shape, lo: float, hi: float) -> np.ndarray:
        return self.rng.uniform(lo, hi, size=shape).astype(np.float32)

    def bn(self, c: int):
        return (self.uniform(c, 0.5, 1.5), self.normal(c, 0.1), self.normal(c, 0.1), self.uniform(c, 0.5, 1.5))


def make_input(shape, seed: int = DEFAULT_SEED, dist: str = "normal") -> np.ndarray:
    """Deterministic synthetic input (seed + 1000 keeps it apart from the weights)."""
    rng = np.random.Generator(np.random.PCG64(seed + 1000))
    if dist == "uniform":
        return rng.uniform(0.0, 1.0, size=shape).astype(np.float32)
    return rng.standard_normal(shape, dtype=np.float64).astype(np.float32)


# ---------------------------------------------------------------------- LeNet

def lenet(seed: int = DEFAULT_SEED) -> Graph:
    p = Params(seed)
    g = Graph("lenet")
    x = g.input("input", [1, 1, 28, 28])
    h = g.relu(g.conv(x, p.he((6, 1, 5, 5)), p.normal(6, 0.01), pad=2))
    h = g.maxpool(h, 2, 2)
    h = g.relu(g.conv(h, p.he((16, 6, 5, 5)), p.normal(16, 0.01)))
    h = g.maxpool(h, 2, 2)
    h = g.flatten(h, 1)
    h = g.relu(g.gemm(h, p.he((120, 400)).T.copy(), p.normal(120, 0.01)))
    h = g.relu(g.gemm(h, p.he((84, 120)).T.copy(), p.normal(84, 0.01)))
    h = g.gemm(h, p.he((10, 84)).T.copy(), p.normal(10, 0.01))
    g.mark_output(g.softmax(h, -1))
    run_default_pipeline(g)
    return g


# --------------------------------------------------------------------- ResNet

def _conv_bn(g: Graph, p: Params, x: int, cout: int, k: int, stride: int, pad: int, relu: bool) -> int:
    cin = g.shape(x)[1]
    h = g.conv(x, p.he((cout, cin, k, k)), None, stride=stride, pad=pad)
    h = g.batchnorm(h, *p.bn(cout))
    return g.relu(h) if relu else h


def _basic_block(g, p, x, width, stride):
    cin = g.shape(x)[1]
    h = _conv_bn(g, p, x, width, 3, stride, 1, True)
    h = _conv_bn(g, p, h, width, 3, 1, 1, False)
    sc = _conv_bn(g, p, x, width, 1, stride, 0, False) if stride != 1 or cin != width else x
    return g.relu(g.add(h, sc))


def _bottleneck(g, p, x, width, stride):
    cin = g.shape(x)[1]
    h = _conv_bn(g, p, x, width, 1, 1, 0, True)
    h = _conv_bn(g, p, h, width, 3, stride, 1, True)
    h = _conv_bn(g, p, h, width * 4, 1, 1, 0, False)
    sc = _conv_bn(g, p, x, width * 4, 1, stride, 0, False) if stride != 1 or cin != width * 4 else x
    return g.relu(g.add(h, sc))


RESNET_STAGES = {18: ("basic", [2, 2, 2, 2]), 50: ("bottleneck", [3, 4, 6, 3]), 101: ("bottleneck", [3, 4, 23, 3])}


def resnet(depth: int, batch: int = 1, seed: int = DEFAULT_SEED, image: int = 224, classes: int = 1000) -> Graph:
    kind, blocks = RESNET_STAGES[depth]
    p = Params(seed)
    g = Graph(f"resnet{depth}")
    x = g.input("input", [batch, 3, image, image])
    h = _conv_bn(g, p, x, 64, 7, 2, 3, True)
    h = g.maxpool(h, 3, 2, 1)
    for stage, (n_blocks, width) in enumerate(zip(blocks, [64, 128, 256, 512])):
        for b in range(n_blocks):
            stride = 2 if (b == 0 and stage > 0) else 1
            h = (_basic_block if kind == "basic" else _bottleneck)(g, p, h, width, stride)
    h = g.reduce_mean(h, [2, 3], keepdims=1)
    h = g.flatten(h, 1)
    c = g.shape(h)[1]
    h = g.gemm(h, p.he((classes, c)).T.copy(), p.normal(classes, 0.01))
    g.mark_output(h)
    run_default_pipeline(g)
    return g


def conv_flops(g: Graph) -> int:
    """Sum of 2*N*Cout*OH*OW*(Cin/g)*KH*KW over Conv nodes."""
    total = 0
    for n in g.nodes:
        if n.op_type != "Conv":
            continue
        y = g.shape(n.outputs[0])
        w = g.tensors[n.inputs[1]].shape
        total += 2 * y[0] * y[1] * y[2] * y[3] * w[1] * w[2] * w[3]
    return total


# --------------------------------------------------------- single-op graphs

def single_conv(n: int, cin: int, h: int, w: int, cout: int, k: int, stride: int = 1, pad: int = 0,
                dilation: int = 1, group: int = 1, act: str | None = "Relu", bias: bool = True,
                residual: bool = False, seed: int = DEFAULT_SEED, pads: list[int] | None = None) -> Graph:
    """One Conv node (after fusion) with optional bias, residual and activation."""
    p = Params(seed)
    g = Graph("conv")
    x = g.input("x", [n, cin, h, w])
    y = g.conv(x, p.he((cout, cin // group, k, k)), p.normal(cout, 0.01) if bias else None, stride=stride,
               pad=pads if pads is not None else pad, dilation=dilation, group=group)
    if residual:
        r = g.input("residual", g.shape(y))
        y = g.add(y, r)
    if act == "Relu":
        y = g.relu(y)
    elif act == "Silu":
        y = g.silu(y)
    g.mark_output(y)
    if residual and act == "Silu":
        raise ValueError("Conv+Add fusion only carries the Add's Relu")
    run_default_pipeline(g)
    return g


def single_gemm(rows: int, k: int, nout: int, *, alpha=1.0, trans_a=0, trans_b=0, bias=True,
                seed=DEFAULT_SEED) -> Graph:
    p = Params(seed)
    g = Graph("gemm")
    a = g.input("a", [k, rows] if trans_a else [rows, k])
    b = p.he((nout, k)) if trans_b else p.he((nout, k)).T.copy()
    y = g.gemm(a, b, p.normal(nout, 0.01) if bias else None, alpha=alpha, trans_a=trans_a, trans_b=trans_b)
    g.mark_output(y)
    return g


def single_op(op: str, shape, **kw) -> Graph:
    """Graphs of one memory-bound op on a random NCHW input."""
    g = Graph(op.lower())
    x = g.input("x", shape)
    if op == "MaxPool":
        y = g.maxpool(x, kw.get("k", 3), kw.get("s", 2), kw.get("p", 1))
    elif op == "AveragePool":
        y = g.avgpool(x, kw.get("k", 3), kw.get("s", 2), kw.get("p", 1))
    elif op == "GlobalAveragePool":
        y = g.global_avgpool(x)
    elif op == "Add":
        b = g.input("b", kw.get("b_shape", shape))
        y = g.add(x, b)
        if kw.get("relu"):
            y = g.relu(y)
            run_default_pipeline(g)
            g.mark_output(g.nodes[-1].outputs[0])
            return g
    elif op in ("Mul", "Sub", "Div", "Mod"):
        b = g.input("b", kw.get("b_shape", shape))
        y = g.binary(op, b, x) if kw.get("swap") else g.binary(op, x, b)
    elif op == "Resize":
        y = g.resize(x, kw.get("scale", 2))
    elif op == "Softmax":
        y = g.softmax(x, kw.get("axis", -1))
    elif op == "ReduceMean":
        y = g.reduce_mean(x, kw.get("axes", [2, 3]), kw.get("keepdims", 1))
    elif op in ("Relu", "Sigmoid"):
        y = g.unary(op, x)
    else:
        raise ValueError(op)
    g.mark_output(y)
    return g


def index_op(op: str, shape, seed: int = DEFAULT_SEED, **kw) -> Graph:
    """Graphs of one indexing / layout op (the YOLO op set) on an input of
    `shape`; index tensors are constants built from `kw`."""
    g = Graph(op.lower())
    x = g.input("x", shape)
    outs: list[int]
    if op == "Transpose":
        outs = [g.transpose(x, kw["perm"])]
    elif op == "Tile":
        outs = [g.tile(x, kw["reps"])]
    elif op == "Split":
        outs = g.split(x, kw["sizes"], kw.get("axis", 1))
    elif op == "Slice":
        outs = [g.slice(x, kw["start"], kw["end"], kw.get("axis", 0), kw.get("step", 1))]
    elif op == "Gather":
        idx = g.weight("indices", np.asarray(kw["indices"], np.float32))
        outs = [g.gather(x, idx, kw.get("axis", 0))]
    elif op == "GatherElements":
        idx = g.weight("indices", np.asarray(kw["indices"], np.float32))
        outs = [g.gather_elements(x, idx, kw.get("axis", 0))]
    elif op == "TopK":
        outs = list(g.topk(x, kw["k"], kw.get("axis", -1), kw.get("largest", 1)))
    elif op == "ReduceMax":
        outs = [g.reduce_max(x, kw["axes"], kw.get("keepdims", 1))]
    else:
        raise ValueError(op)
    for t in outs:
        g.mark_output(t)
    return g


def matmul_op(a_shape, b_shape, const_b: bool = False, seed: int = DEFAULT_SEED) -> Graph:
    """One batched MatMul with numpy-style broadcasting of the leading dims;
    B is a second input, or a constant weight with `const_b`."""
    g = Graph("matmul")
    a = g.input("a", list(a_shape))
    if const_b:
        b = g.weight("b", Params(seed).normal(tuple(b_shape), 0.5))
    else:
        b = g.input("b", list(b_shape))
    g.mark_output(g.matmul(a, b))
    return g


# ------------------------------------------------------- YOLOv10n-style graph

def _cbs(g: Graph, p: Params, x: int, cout: int, k: int, stride: int = 1) -> int:
    """Conv + BN + SiLU (the SiLU as Sigmoid*Mul, fused by the pipeline)."""
    cin = g.shape(x)[1]
    h = g.conv(x, p.he((cout, cin, k, k)), None, stride=stride, pad=k // 2)
    h = g.batchnorm(h, *p.bn(cout))
    return g.silu(h)


def _c2f(g: Graph, p: Params, x: int, c: int, n: int, shortcut: bool = True) -> int:
    """CSP bottleneck with two convs: 1x1, Split in halves, n residual
    bottlenecks on the second half (standalone Adds: the convs carry SiLU),
    Concat of every branch, 1x1."""
    h = _cbs(g, p, x, c, 1)
    a, b = g.split(h, [c // 2, c // 2], axis=1)
    parts = [a, b]
    for _ in range(n):
        t = _cbs(g, p, parts[-1], c // 2, 3)
        t = _cbs(g, p, t, c // 2, 3)
        parts.append(g.add(parts[-1], t) if shortcut else t)
    return _cbs(g, p, g.concat(parts, axis=1), c, 1)


def _sppf(g: Graph, p: Params, x: int, c: int) -> int:
    h = _cbs(g, p, x, c // 2, 1)
    y1 = g.maxpool(h, 5, 1, 2)
    y2 = g.maxpool(y1, 5, 1, 2)
    y3 = g.maxpool(y2, 5, 1, 2)
    return _cbs(g, p, g.concat([h, y1, y2, y3], axis=1), c, 1)


def _cb(g: Graph, p: Params, x: int, cout: int, k: int = 1, group: int = 1) -> int:
    """Conv + BN without activation."""
    cin = g.shape(x)[1]
    h = g.conv(x, p.he((cout, cin // group, k, k)), None, pad=k // 2, group=group)
    return g.batchnorm(h, *p.bn(cout))


def _attention(g: Graph, p: Params, x: int, heads: int) -> int:
    """Multi-head self-attention over the H*W positions of a feature map
    (YOLOv10's PSA attention): 1x1 qkv projection with keys half the head
    width, softmax((q^T k) / sqrt(key_dim)) over keys, v weighted by the
    attention, plus a depthwise 3x3 positional term on v, 1x1 output
    projection."""
    b, dim, hh, ww = g.shape(x)
    n = hh * ww
    head_dim = dim // heads
    key_dim = head_dim // 2
    qkv = _cb(g, p, x, dim + 2 * key_dim * heads)
    qkv = g.reshape(qkv, [b, heads, 2 * key_dim + head_dim, n])
    q, k, v = g.split(qkv, [key_dim, key_dim, head_dim], axis=2)
    attn = g.matmul(g.transpose(q, [0, 1, 3, 2]), k)                      # [b, heads, n, n]
    attn = g.binary("Mul", attn, g._const("attn_scale", [key_dim ** -0.5]))
    attn = g.softmax(attn, axis=-1)
    out = g.matmul(v, g.transpose(attn, [0, 1, 3, 2]))                    # [b, heads, head_dim, n]
    out = g.reshape(out, [b, dim, hh, ww])
    pe = _cb(g, p, g.reshape(v, [b, dim, hh, ww]), dim, 3, group=dim)
    return _cb(g, p, g.add(out, pe), dim)


def _psa(g: Graph, p: Params, x: int, c: int) -> int:
    """Partial self-attention block: 1x1, split in halves, attention and a
    two-conv feed-forward (each residual) on the second half, concat, 1x1."""
    h = _cbs(g, p, x, c, 1)
    a, b = g.split(h, [c // 2, c // 2], axis=1)
    b = g.add(b, _attention(g, p, b, max(1, c // 128)))
    b = g.add(b, _cb(g, p, _cbs(g, p, b, c, 1), c // 2))
    return _cbs(g, p, g.concat([a, b], axis=1), c, 1)


def yolo_v10n(batch: int = 1, image: int = 640, seed: int = DEFAULT_SEED, classes: int = 80,
              topk: int = 300) -> Graph:
    """YOLOv10n-style detector: CSP backbone of 3x3/2
    Conv+BN+SiLU downsamples 16->32->64->128->256 with C2f split/concat
    blocks, SPPF, a PSA attention block (2 heads over the stride-32 map:
    batched MatMul, Softmax), PAN neck (nearest Resize x2 + Concat), decoupled heads at
    strides 8/16/32 (4x16 box bins + `classes` scores), and the pre-NMS
    post-processing: DFL Softmax over the 16 bins, class Sigmoid, per-anchor
    max, TopK(`topk`), GatherElements of boxes and scores.  Outputs: top
    scores [B, k], boxes [B, k, 4] (DFL expectations), class scores
    [B, k, classes], anchor indices [B, k]."""
    p = Params(seed)
    g = Graph("yolov10n")
    x = g.input("images", [batch, 3, image, image])
    h = _cbs(g, p, x, 16, 3, 2)
    h = _cbs(g, p, h, 32, 3, 2)
    h = _c2f(g, p, h, 32, 1)
    h = _cbs(g, p, h, 64, 3, 2)
    p3 = _c2f(g, p, h, 64, 2)
    h = _cbs(g, p, p3, 128, 3, 2)
    p4 = _c2f(g, p, h, 128, 2)
    h = _cbs(g, p, p4, 256, 3, 2)
    h = _c2f(g, p, h, 256, 1)
    p5 = _psa(g, p, _sppf(g, p, h, 256), 256)
    # PAN neck
    n4 = _c2f(g, p, g.concat([g.resize(p5, 2), p4], axis=1), 128, 1, shortcut=False)
    n3 = _c2f(g, p, g.concat([g.resize(n4, 2), p3], axis=1), 64, 1, shortcut=False)
    o4 = _c2f(g, p, g.concat([_cbs(g, p, n3, 64, 3, 2), n4], axis=1), 128, 1, shortcut=False)
    o5 = _c2f(g, p, g.concat([_cbs(g, p, o4, 128, 3, 2), p5], axis=1), 256, 1, shortcut=False)
    # decoupled heads
    bins = 16
    levels = []
    for feat in (n3, o4, o5):
        box = _cbs(g, p, _cbs(g, p, feat, 64, 3), 64, 3)
        box = g.conv(box, p.he((4 * bins, 64, 1, 1)), p.normal(4 * bins, 0.01))
        cls = _cbs(g, p, _cbs(g, p, feat, classes, 3), classes, 3)
        cls = g.conv(cls, p.he((classes, classes, 1, 1)), p.normal(classes, 0.01))
        hw = g.shape(box)[2] * g.shape(box)[3]
        levels.append(g.reshape(g.concat([box, cls], axis=1), [batch, 4 * bins + classes, hw]))
    out = g.concat(levels, axis=2)  # [B, 64 + classes, A]
    anchors = g.shape(out)[2]
    box, cls = g.split(out, [4 * bins, classes], axis=1)
    # DFL: softmax over the 16 bins of each side, expectation by a 1x1 conv
    box = g.transpose(g.reshape(box, [batch, 4, bins, anchors]), [0, 2, 1, 3])  # [B, 16, 4, A]
    box = g.softmax(box, axis=1)
    dfl = g.conv(box, np.arange(bins, dtype=np.float32).reshape(1, bins, 1, 1), None)  # [B, 1, 4, A]
    dist = g.transpose(g.reshape(dfl, [batch, 4, anchors]), [0, 2, 1])  # [B, A, 4]
    scores = g.transpose(g.unary("Sigmoid", cls), [0, 2, 1])  # [B, A, classes]
    best = g.reduce_max(scores, [2], keepdims=0)  # [B, A]
    k = min(topk, anchors)
    top_v, top_i = g.topk(best, k, axis=1, largest=1)
    idx = g.unsqueeze(top_i, 2)  # [B, k, 1]
    boxes = g.gather_elements(dist, g.tile(idx, [1, 1, 4]), axis=1)
    cls_k = g.gather_elements(scores, g.tile(idx, [1, 1, classes]), axis=1)
    for t in (top_v, boxes, cls_k, top_i):
        g.mark_output(t)
    run_default_pipeline(g)
    return g
