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


def single_gemm(rows: int, k: int, nout: int, *, alpha=1.0, trans_b=0, bias=True, seed=DEFAULT_SEED) -> Graph:
    p = Params(seed)
    g = Graph("gemm")
    a = g.input("a", [rows, k])
    b = p.he((nout, k)) if trans_b else p.he((nout, k)).T.copy()
    y = g.gemm(a, b, p.normal(nout, 0.01) if bias else None, alpha=alpha, trans_b=trans_b)
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
    elif op in ("Mul", "Sub", "Div"):
        b = g.input("b", kw.get("b_shape", shape))
        y = g.binary(op, x, b)
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
