"""Runs an SPK package on the CPU oracle (oracle/liboracle.so), node by node.

TEST INFRASTRUCTURE ONLY: the checker the parity tests compare the MI355X
runtime against.  It parses the package with its own minimal reader (not the
product's loader or writer), keeps every tensor as a separate numpy array (so
a wrong arena plan in the product shows up as a mismatch), and calls the C
restatement of each reference kernel.  Dispatch order and per-op semantics
follow the reference executor (runtime/core/executor.c:500-537) and kernels.
"""

from __future__ import annotations

import ctypes
import json
import struct
from dataclasses import dataclass
from pathlib import Path

import numpy as np

ORACLE_LIB = Path(__file__).resolve().parent / "liboracle.so"

_HDR = struct.Struct("<IHHHHIIIIIIQQQII")
_SEC = struct.Struct("<IIQQII")
_TEN = struct.Struct("<IHHHH8IQQII")
_NODE = struct.Struct("<IHHHH8I4IIIII")
_ATTR = struct.Struct("<Iiii4i2i2i2i2i2fii8i3i")
_QP = struct.Struct("<IHHIQ")

OPS = {1: "Add", 2: "Conv", 3: "Flatten", 4: "Gemm", 5: "MaxPool", 6: "Relu", 7: "Softmax", 8: "Mul", 9: "Sub",
       10: "Div", 11: "Mod", 12: "Sigmoid", 13: "Reshape", 14: "Transpose", 15: "Concat", 16: "Split",
       17: "ReduceMean", 18: "ReduceMax", 19: "MatMul", 20: "Resize", 21: "Tile", 22: "Unsqueeze",
       23: "GatherElements", 24: "TopK", 25: "Cast", 26: "Slice", 27: "Gather", 28: "AveragePool",
       29: "GlobalAveragePool"}


@dataclass
class TensorInfo:
    id: int
    dtype: int
    role: int
    shape: tuple
    size: int
    offset: int


@dataclass
class NodeInfo:
    id: int
    op: int
    inputs: list
    outputs: list
    attr: dict


def _lib():
    if not ORACLE_LIB.exists():
        raise FileNotFoundError(f"{ORACLE_LIB} not built (make -C oracle oracle)")
    lib = ctypes.CDLL(str(ORACLE_LIB))
    return lib


class Package:
    """Minimal independent reader of an SPK v0.3 blob."""

    def __init__(self, blob: bytes) -> None:
        h = _HDR.unpack_from(blob, 0)
        assert h[0] == 0x32564B50, "bad magic"
        self.num_tensors, self.num_nodes = h[7], h[8]
        secs = {}
        for i in range(h[5]):
            kind, _, off, size, _, _ = _SEC.unpack_from(blob, h[4] + i * _SEC.size)
            secs[kind] = (off, size)
        toff = secs[3][0]
        self.tensors = []
        for i in range(self.num_tensors):
            f = _TEN.unpack_from(blob, toff + i * _TEN.size)
            self.tensors.append(TensorInfo(f[0], f[1], f[2], tuple(f[5:5 + f[3]]), f[13], f[14]))
        noff = secs[4][0]
        aoff = secs[5][0]
        self.nodes = []
        for i in range(self.num_nodes):
            f = _NODE.unpack_from(blob, noff + i * _NODE.size)
            nin, nout = f[3], f[4]
            a = _ATTR.unpack_from(blob, aoff + f[17])
            attr = dict(op=a[0], axis=a[1], group=a[2], act=a[3], pads=a[4:8], strides=a[8:10], kernel=a[10:12],
                        dil=a[12:14], trans_a=a[14], trans_b=a[15], alpha=a[16], beta=a[17], extra_count=a[18],
                        keepdims=a[19], extra=a[20:28], largest=a[28], sorted=a[29], cast_to=a[30])
            self.nodes.append(NodeInfo(f[0], f[1], list(f[5:5 + nin]), list(f[13:13 + nout]), attr))
        woff = secs[6][0]
        self.weights = {}
        for t in self.tensors:
            if t.role == 3:
                raw = blob[woff + t.offset: woff + t.offset + t.size]
                # dtype 3: IEEE half weights, widened exactly to fp32 (reference
                # runtime/kernels/optimized/conv/conv.c:961-978)
                dt = {2: np.int8, 3: np.dtype("<f2")}.get(t.dtype, np.dtype("<f4"))
                w = np.frombuffer(raw, dtype=dt).reshape(t.shape)
                self.weights[t.id] = w.astype(np.float32) if t.dtype == 3 else w.copy()
        self.quant = {}
        self.zero_points = {}
        if 9 in secs:
            qoff, qsize = secs[9]
            first = _QP.unpack_from(blob, qoff)
            count = first[4] // _QP.size
            for i in range(count):
                tid, scheme, axis, nch, doff = _QP.unpack_from(blob, qoff + i * _QP.size)
                self.quant[tid] = np.frombuffer(blob[qoff + doff: qoff + doff + 4 * nch], dtype="<f4").copy()
                # int32 zero points follow the scales (reference spk_writer.py quantization section)
                zoff = qoff + doff + 4 * nch
                self.zero_points[tid] = np.frombuffer(blob[zoff: zoff + 4 * nch], dtype="<i4").copy()
        meta = json.loads(blob[secs[1][0]: secs[1][0] + secs[1][1]].decode())
        self.inputs = [t.id for t in self.tensors if t.role == 1]
        self.outputs = list(meta.get("outputs", [t.id for t in self.tensors if t.role == 2]))


def _f(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p) if a is not None else None


class OracleExecutor:
    def __init__(self, blob: bytes) -> None:
        self.pkg = Package(blob)
        self.lib = _lib()
        self.acc: dict[int, np.ndarray] = {}  # int8 conv node id -> int32 accumulators of the last run

    def run(self, *inputs: np.ndarray, keep: bool = False) -> list[np.ndarray] | dict[int, np.ndarray]:
        pkg = self.pkg
        vals: dict[int, np.ndarray] = dict(pkg.weights)
        for tid, x in zip(pkg.inputs, inputs):
            vals[tid] = np.ascontiguousarray(x, dtype=np.float32).reshape(pkg.tensors[tid].shape)
        for n in pkg.nodes:
            op = OPS.get(n.op)
            if op is None:
                raise NotImplementedError(f"oracle has no op code {n.op}")
            getattr(self, "_" + op.lower())(n, vals)
        if keep:
            return vals
        return [vals[t] for t in pkg.outputs]

    # ------------------------------------------------------------------ ops
    def _shape(self, tid):
        return self.pkg.tensors[tid].shape

    def _out(self, n, vals, dtype=np.float32):
        y = np.zeros(self._shape(n.outputs[0]), dtype=dtype)
        vals[n.outputs[0]] = y
        return y

    def _is_q8(self, tid) -> bool:
        """An int8 activation tensor (the INT8 configuration with int8
        tensors between nodes)."""
        t = self.pkg.tensors[tid]
        return t.dtype == 2 and t.role != 3

    def _qz(self, tid):
        return float(self.pkg.quant[tid][0]), int(self.pkg.zero_points[tid][0])

    def _conv_q8(self, n, vals):
        """Conv of the INT8 configuration (spk_oracle.c oracle_q8_conv): int8
        (or fp32, quantized on load) input with (s_x, z_x), per-channel int8
        weights, int32 accumulation, fixed-point requantization into int8
        with (s_y, z_y), int8 residual with (s_r, z_r), Relu clamp."""
        lib = self.lib
        x = vals[n.inputs[0]]
        w = vals[n.inputs[1]]
        b = vals[n.inputs[2]] if len(n.inputs) > 2 else None
        sx, zx = self._qz(n.inputs[0])
        sy, zy = self._qz(n.outputs[0])
        if x.dtype != np.int8:
            xf = np.ascontiguousarray(x, dtype=np.float32)
            x = np.zeros(xf.shape, np.int8)
            lib.oracle_q8_quantize(_f(xf), _f(x), ctypes.c_size_t(xf.size), ctypes.c_float(sx), zx)
        r, sr, zr = None, 0.0, 0
        if len(n.inputs) > 3:
            r = np.ascontiguousarray(vals[n.inputs[3]])
            assert r.dtype == np.int8, "the INT8 configuration's residual is an int8 tensor"
            sr, zr = self._qz(n.inputs[3])
        M = w.shape[0]
        sw = np.ascontiguousarray(self.pkg.quant[n.inputs[1]][:M], dtype=np.float32)
        bq, m1, m2, shf = (np.zeros(M, np.int32) for _ in range(4))
        rc = lib.oracle_q8_requant_params(ctypes.c_float(sx), _f(sw), ctypes.c_float(sy), ctypes.c_float(sr),
                                          _f(np.ascontiguousarray(b, dtype=np.float32) if b is not None else None),
                                          M, _f(bq), _f(m1), _f(m2), _f(shf))
        assert rc == 0, "requantization shift out of range"
        y = self._out(n, vals, np.int8)
        acc = np.zeros(y.shape, np.int32)
        N, C, H, W = x.shape
        _, _, KH, KW = w.shape
        a = n.attr
        lib.oracle_q8_conv(_f(np.ascontiguousarray(x)), zx, _f(w), _f(bq), _f(m1), _f(m2), _f(shf), _f(r), zr, zy,
                           int(a["act"] == 1), _f(y), _f(acc), N, C, H, W, M, KH, KW, y.shape[2], y.shape[3],
                           a["strides"][0], a["strides"][1], a["pads"][0], a["pads"][1], a["dil"][0], a["dil"][1])
        self.acc[n.id] = acc

    def _conv(self, n, vals):
        if self._is_q8(n.outputs[0]) or self._is_q8(n.inputs[0]):
            return self._conv_q8(n, vals)
        x = vals[n.inputs[0]]
        w = vals[n.inputs[1]]
        b = vals[n.inputs[2]] if len(n.inputs) > 2 else None
        r = np.ascontiguousarray(vals[n.inputs[3]]) if len(n.inputs) > 3 else None
        y = self._out(n, vals)
        N, C, H, W = x.shape
        M, _, KH, KW = w.shape
        OH, OW = y.shape[2], y.shape[3]
        a = n.attr
        geo = (N, C, H, W, M, KH, KW, OH, OW, a["strides"][0], a["strides"][1], a["pads"][0], a["pads"][1],
               a["dil"][0], a["dil"][1])
        if w.dtype == np.int8:
            ws = self.pkg.quant[n.inputs[1]]
            xs = self.pkg.quant[n.inputs[0]][0]
            acc = np.zeros(y.shape, dtype=np.int32)
            rc = self.lib.oracle_conv2d_int8(_f(x), _f(w), _f(ws), ctypes.c_float(xs), _f(b), _f(r), _f(y), _f(acc),
                                             *geo, a["act"])
            self.acc[n.id] = acc
        else:
            rc = self.lib.oracle_conv2d_f32(_f(x), _f(w), _f(b), _f(r), _f(y), *geo, a["group"], a["act"])
        assert rc == 0, rc

    def _gemm(self, n, vals):
        a_, b_ = vals[n.inputs[0]], vals[n.inputs[1]]
        c = vals[n.inputs[2]] if len(n.inputs) > 2 else None
        y = self._out(n, vals)
        at = n.attr["trans_a"]
        rows = a_.shape[1] if at else a_.shape[0]
        k = a_.shape[0] if at else a_.shape[1]
        nout = b_.shape[0] if n.attr["trans_b"] else b_.shape[1]
        self.lib.oracle_gemm_f32(_f(a_), _f(b_), _f(c), _f(y), rows, k, nout, at, n.attr["trans_b"],
                                 ctypes.c_float(n.attr["alpha"]))

    def _matmul(self, n, vals):
        a_, b_ = vals[n.inputs[0]], vals[n.inputs[1]]
        y = self._out(n, vals)
        M, N = y.shape[-2], y.shape[-1]
        K = a_.shape[-1]
        lead = y.shape[:-2]
        ai = np.broadcast_to(np.arange(int(np.prod(a_.shape[:-2]))).reshape(a_.shape[:-2] or (1,)), lead or (1,))
        bi = np.broadcast_to(np.arange(int(np.prod(b_.shape[:-2]))).reshape(b_.shape[:-2] or (1,)), lead or (1,))
        aoff = np.ascontiguousarray(ai.reshape(-1) * M * K, dtype=np.int64)
        boff = np.ascontiguousarray(bi.reshape(-1) * K * N, dtype=np.int64)
        self.lib.oracle_matmul_f32(_f(a_), _f(b_), _f(y), len(aoff), _f(aoff), _f(boff), M, K, N)

    def _pool_args(self, n, vals):
        x = vals[n.inputs[0]]
        y = self._out(n, vals)
        a = n.attr
        return x, y, (*x.shape, y.shape[2], y.shape[3], a["kernel"][0], a["kernel"][1], a["strides"][0],
                      a["strides"][1], a["pads"][0], a["pads"][1])

    def _maxpool(self, n, vals):
        if vals[n.inputs[0]].dtype == np.int8:
            assert self._is_q8(n.outputs[0]) and self._qz(n.inputs[0]) == self._qz(n.outputs[0])
            x = vals[n.inputs[0]]
            y = self._out(n, vals, np.int8)
            a = n.attr
            self.lib.oracle_q8_maxpool(_f(x), _f(y), *x.shape, y.shape[2], y.shape[3], a["kernel"][0],
                                       a["kernel"][1], a["strides"][0], a["strides"][1], a["pads"][0], a["pads"][1])
            return
        x, y, g = self._pool_args(n, vals)
        self.lib.oracle_maxpool_f32(_f(x), _f(y), *g)

    def _plane_mean_q8(self, n, vals):
        x = vals[n.inputs[0]]
        y = self._out(n, vals)
        s, z = self._qz(n.inputs[0])
        self.lib.oracle_q8_plane_mean(_f(x), _f(y), ctypes.c_size_t(x.shape[0] * x.shape[1]), x.shape[2] * x.shape[3],
                                      ctypes.c_float(s), z)

    def _averagepool(self, n, vals):
        x, y, g = self._pool_args(n, vals)
        self.lib.oracle_avgpool_f32(_f(x), _f(y), *g)

    def _globalaveragepool(self, n, vals):
        if vals[n.inputs[0]].dtype == np.int8:
            return self._plane_mean_q8(n, vals)
        x = vals[n.inputs[0]]
        y = self._out(n, vals)
        self.lib.oracle_global_avgpool_f32(_f(x), _f(y), x.shape[0], x.shape[1], x.shape[2] * x.shape[3])

    def _binary(self, n, vals, code):
        a_, b_ = vals[n.inputs[0]], vals[n.inputs[1]]
        y = self._out(n, vals)
        sh = lambda t: (ctypes.c_uint32 * 8)(*t.shape)  # noqa: E731
        rc = self.lib.oracle_binary_f32(code, _f(a_), sh(a_), a_.ndim, _f(b_), sh(b_), b_.ndim, _f(y), sh(y), y.ndim,
                                        n.attr["act"] if code == 1 else 0)
        assert rc == 0

    def _add(self, n, vals):
        self._binary(n, vals, 1)

    def _mul(self, n, vals):
        self._binary(n, vals, 8)

    def _sub(self, n, vals):
        self._binary(n, vals, 9)

    def _div(self, n, vals):
        self._binary(n, vals, 10)

    def _mod(self, n, vals):
        self._binary(n, vals, 11)

    def _relu(self, n, vals):
        x = vals[n.inputs[0]]
        y = self._out(n, vals)
        self.lib.oracle_relu_f32(_f(x), _f(y), ctypes.c_size_t(x.size))

    def _sigmoid(self, n, vals):
        x = vals[n.inputs[0]]
        y = self._out(n, vals)
        self.lib.oracle_sigmoid_f32(_f(x), _f(y), ctypes.c_size_t(x.size))

    def _softmax(self, n, vals):
        x = vals[n.inputs[0]]
        y = self._out(n, vals)
        ax = n.attr["axis"] % x.ndim
        outer = int(np.prod(x.shape[:ax]))
        inner = int(np.prod(x.shape[ax + 1:]))
        self.lib.oracle_softmax_f32(_f(x), _f(y), ctypes.c_size_t(outer), ctypes.c_size_t(x.shape[ax]),
                                    ctypes.c_size_t(inner))

    def _reduce(self, n, vals, is_max):
        x = vals[n.inputs[0]]
        y = self._out(n, vals)
        a = n.attr
        if a["extra_count"] > 0:
            axes = [v % x.ndim for v in a["extra"][:a["extra_count"]]]
        else:
            axes = list(range(x.ndim))
        mask = 0
        for ax in axes:
            mask |= 1 << ax
        shp = (ctypes.c_uint32 * 8)(*x.shape)
        self.lib.oracle_reduce_f32(_f(x), shp, x.ndim, ctypes.c_uint32(mask), int(is_max), _f(y))

    def _reducemean(self, n, vals):
        x = vals[n.inputs[0]]
        if x.dtype == np.int8:
            a = n.attr
            axes = sorted(v % x.ndim for v in a["extra"][:a["extra_count"]])
            assert x.ndim == 4 and axes == [2, 3], "int8 ReduceMean over the spatial axes only"
            return self._plane_mean_q8(n, vals)
        self._reduce(n, vals, False)

    def _reducemax(self, n, vals):
        self._reduce(n, vals, True)

    def _resize(self, n, vals):
        x = vals[n.inputs[0]]
        y = self._out(n, vals)
        self.lib.oracle_resize_nearest_f32(_f(x), _f(y), *x.shape, y.shape[2], y.shape[3])

    def _copy(self, n, vals):
        vals[n.outputs[0]] = vals[n.inputs[0]].reshape(self._shape(n.outputs[0])).copy()

    _flatten = _reshape = _unsqueeze = _cast = _copy

    def _concat(self, n, vals):
        ax = n.attr["axis"] % len(self._shape(n.outputs[0]))
        vals[n.outputs[0]] = np.concatenate([vals[t] for t in n.inputs], axis=ax)

    # ---- indexing / layout (integer index arithmetic, restated with numpy) ----
    def _transpose(self, n, vals):
        # reference shape/transpose.c:14-18: x coord perm[d] = y coord d
        x = vals[n.inputs[0]]
        a = n.attr
        perm = list(a["extra"][:a["extra_count"]]) if a["extra_count"] > 0 else list(range(x.ndim))
        vals[n.outputs[0]] = np.ascontiguousarray(np.transpose(x, perm))

    def _tile(self, n, vals):
        # reference shape/tile.c:13-19: x coord = y coord mod x dim
        x = vals[n.inputs[0]]
        y_shape = self._shape(n.outputs[0])
        idx = np.ix_(*[np.arange(ys) % xs for ys, xs in zip(y_shape, x.shape)])
        vals[n.outputs[0]] = np.ascontiguousarray(x[idx])

    def _split(self, n, vals):
        # reference tensor/split.c:15-27: consecutive blocks along axis
        x = vals[n.inputs[0]]
        ax = n.attr["axis"] % x.ndim
        start = 0
        for t in n.outputs:
            size = self._shape(t)[ax]
            vals[t] = np.ascontiguousarray(np.take(x, np.arange(start, start + size), axis=ax))
            start += size

    def _slice(self, n, vals):
        # reference tensor/slice.c:12-49, first value of each parameter tensor
        x = vals[n.inputs[0]]
        start = int(vals[n.inputs[1]].ravel()[0])
        end = int(vals[n.inputs[2]].ravel()[0])
        axis = int(vals[n.inputs[3]].ravel()[0]) if len(n.inputs) > 3 else 0
        step = int(vals[n.inputs[4]].ravel()[0]) if len(n.inputs) > 4 else 1
        if axis < 0:
            axis += x.ndim
        dim = x.shape[axis]
        if start < 0:
            start += dim
        if end < 0:
            end += dim
        if end > dim:
            end = dim
        if start < 0:
            start = 0
        out = (end - start + step - 1) // step
        vals[n.outputs[0]] = np.ascontiguousarray(np.take(x, start + step * np.arange(out), axis=axis))

    def _gather(self, n, vals):
        # reference tensor/gather.c:28-36: (int)index, negative + dim
        data, idx = vals[n.inputs[0]], vals[n.inputs[1]]
        ax = n.attr["axis"] % data.ndim
        ix = idx.astype(np.float32).astype(np.int64)  # C float -> int truncates
        ix = np.where(ix < 0, ix + data.shape[ax], ix)
        vals[n.outputs[0]] = np.ascontiguousarray(np.take(data, ix, axis=ax)).reshape(self._shape(n.outputs[0]))

    def _gatherelements(self, n, vals):
        # reference tensor/gather_elements.c:17-25
        data, idx = vals[n.inputs[0]], vals[n.inputs[1]]
        ax = n.attr["axis"] % data.ndim
        ix = idx.astype(np.int64)
        ix = np.where(ix < 0, ix + data.shape[ax], ix)
        vals[n.outputs[0]] = np.ascontiguousarray(np.take_along_axis(data, ix, axis=ax))

    def _topk(self, n, vals):
        # reference tensor/topk.c via oracle_topk_row, one (outer, inner) row at a time
        x = np.ascontiguousarray(vals[n.inputs[0]], dtype=np.float32)
        k = int(vals[n.inputs[1]].ravel()[0])
        ax = n.attr["axis"] % x.ndim
        dim = x.shape[ax]
        k = min(k, dim)
        outer = int(np.prod(x.shape[:ax]))
        inner = int(np.prod(x.shape[ax + 1:]))
        values = np.zeros(self._shape(n.outputs[0]), np.float32)
        indices = np.zeros(self._shape(n.outputs[1]), np.float32)
        xv, vv, iv = x.reshape(outer, dim, inner), values.reshape(outer, k, inner), indices.reshape(outer, k, inner)
        fp = ctypes.POINTER(ctypes.c_float)
        for o in range(outer):
            for i in range(inner):
                # the C routine walks the row with stride `inner`
                self.lib.oracle_topk_row(
                    ctypes.cast(xv.ctypes.data + 4 * (o * dim * inner + i), fp), ctypes.c_size_t(inner), dim, k,
                    int(n.attr["largest"] != 0),
                    ctypes.cast(vv.ctypes.data + 4 * (o * k * inner + i), fp),
                    ctypes.cast(iv.ctypes.data + 4 * (o * k * inner + i), fp))
        vals[n.outputs[0]] = values
        vals[n.outputs[1]] = indices


def _setup_signatures() -> None:
    pass
