"""Programmatic graph construction with ONNX-style shape inference.

The reference compiler loads ONNX files through onnx + onnxsim
(frontend/onnx_loader.py:47-168). Neither package is importable in this
environment, so graphs are also built in code: each method appends one node
with ONNX attribute names and infers the output shape as ONNX would.
"""

from __future__ import annotations

import numpy as np

from .ir import Graph, Node, TensorInfo


class GraphBuilder:
    def __init__(self, name: str = "model"):
        self.g = Graph(name)
        self._count: dict[str, int] = {}

    # -- naming ------------------------------------------------------------
    def _name(self, prefix: str) -> str:
        k = self._count.get(prefix, 0)
        self._count[prefix] = k + 1
        return f"{prefix}_{k}" if k else prefix

    def _out(self, prefix: str, shape, dtype="float32", name: str | None = None) -> str:
        n = name or self._name(f"{prefix}_output")
        self.g.add_tensor(TensorInfo(n, tuple(int(s) for s in shape), dtype))
        return n

    def _node(self, op, inputs, outputs, name=None, **attrs) -> Node:
        node = Node(name or self._name(f"/{op}"), op, list(inputs), list(outputs), dict(attrs))
        self.g.add_node(node)
        return node

    def shape(self, t: str) -> tuple:
        return self.g.tensors[t].shape

    # -- graph I/O -----------------------------------------------------------
    def input(self, name: str, shape, dtype="float32") -> str:
        self.g.add_tensor(TensorInfo(name, tuple(shape), dtype))
        self.g.inputs.append(name)
        return name

    def const(self, name: str, array: np.ndarray) -> str:
        a = np.ascontiguousarray(array)
        self.g.add_tensor(TensorInfo(name, tuple(a.shape), a.dtype.name, a))
        return name

    def output(self, t: str) -> str:
        self.g.outputs.append(t)
        return t

    def build(self) -> Graph:
        return self.g

    # -- convolution / pooling --------------------------------------------------
    def conv(self, x, w, b=None, strides=(1, 1), pads=(0, 0, 0, 0), name=None, out=None) -> str:
        n, _, h, wd = self.shape(x)
        co, _, kh, kw = self.shape(w)
        ho = (h + pads[0] + pads[2] - kh) // strides[0] + 1
        wo = (wd + pads[1] + pads[3] - kw) // strides[1] + 1
        y = self._out(name or "conv", (n, co, ho, wo), name=out)
        ins = [x, w] + ([b] if b is not None else [])
        self._node("Conv", ins, [y], name, kernel_shape=[kh, kw], strides=list(strides), pads=list(pads))
        return y

    def _pool(self, op, x, kernel, strides, pads, name, out):
        n, c, h, w = self.shape(x)
        ho = (h + pads[0] + pads[2] - kernel[0]) // strides[0] + 1
        wo = (w + pads[1] + pads[3] - kernel[1]) // strides[1] + 1
        y = self._out(name or op.lower(), (n, c, ho, wo), name=out)
        self._node(op, [x], [y], name, kernel_shape=list(kernel), strides=list(strides), pads=list(pads))
        return y

    def maxpool(self, x, kernel=(2, 2), strides=(2, 2), pads=(0, 0, 0, 0), name=None, out=None):
        return self._pool("MaxPool", x, kernel, strides, pads, name, out)

    def avgpool(self, x, kernel=(2, 2), strides=(2, 2), pads=(0, 0, 0, 0), name=None, out=None):
        return self._pool("AveragePool", x, kernel, strides, pads, name, out)

    def global_avgpool(self, x, name=None, out=None):
        n, c, _, _ = self.shape(x)
        y = self._out(name or "gap", (n, c, 1, 1), name=out)
        self._node("GlobalAveragePool", [x], [y], name)
        return y

    # -- element-wise ----------------------------------------------------------
    def _unary(self, op, x, name=None, out=None, **attrs):
        y = self._out(name or op.lower(), self.shape(x), self.g.tensors[x].dtype, name=out)
        self._node(op, [x], [y], name, **attrs)
        return y

    def relu(self, x, name=None, out=None):
        return self._unary("Relu", x, name, out)

    def sigmoid(self, x, name=None, out=None):
        return self._unary("Sigmoid", x, name, out)

    def tanh(self, x, name=None, out=None):
        return self._unary("Tanh", x, name, out)

    def sqrt(self, x, name=None, out=None):
        return self._unary("Sqrt", x, name, out)

    def exp(self, x, name=None, out=None):
        return self._unary("Exp", x, name, out)

    def clip(self, x, lo=None, hi=None, name=None, out=None):
        attrs = {}
        if lo is not None:
            attrs["min"] = float(lo)
        if hi is not None:
            attrs["max"] = float(hi)
        return self._unary("Clip", x, name, out, **attrs)

    def identity(self, x, name=None, out=None):
        return self._unary("Identity", x, name, out)

    def _binary(self, op, a, b, name=None, out=None):
        sa, sb = self.shape(a), self.shape(b)
        shape = tuple(np.broadcast_shapes(sa, sb))
        y = self._out(name or op.lower(), shape, name=out)
        self._node(op, [a, b], [y], name)
        return y

    def add(self, a, b, name=None, out=None):
        return self._binary("Add", a, b, name, out)

    def sub(self, a, b, name=None, out=None):
        return self._binary("Sub", a, b, name, out)

    def mul(self, a, b, name=None, out=None):
        return self._binary("Mul", a, b, name, out)

    def div(self, a, b, name=None, out=None):
        return self._binary("Div", a, b, name, out)

    # -- matrix products ---------------------------------------------------------
    def gemm(self, a, b, c=None, alpha=1.0, beta=1.0, transA=0, transB=0, name=None, out=None):
        sa, sb = self.shape(a), self.shape(b)
        m = sa[1] if transA else sa[0]
        nn = sb[0] if transB else sb[1]
        y = self._out(name or "gemm", (m, nn), name=out)
        ins = [a, b] + ([c] if c is not None else [])
        self._node("Gemm", ins, [y], name, alpha=float(alpha), beta=float(beta), transA=int(transA),
                   transB=int(transB))
        return y

    def matmul(self, a, b, name=None, out=None):
        sa, sb = self.shape(a), self.shape(b)
        if len(sa) == 1 and len(sb) == 2:
            shape = (sb[1],)
        elif len(sa) == 2 and len(sb) == 1:
            shape = (sa[0],)
        else:
            batch = np.broadcast_shapes(tuple(sa[:-2]), tuple(sb[:-2]))
            shape = tuple(batch) + (sa[-2], sb[-1])
        y = self._out(name or "matmul", shape, name=out)
        self._node("MatMul", [a, b], [y], name)
        return y

    # -- normalisation / reductions ----------------------------------------------
    def softmax(self, x, axis=-1, name=None, out=None):
        return self._unary("Softmax", x, name, out, axis=int(axis))

    def layernorm(self, x, scale=None, bias=None, axis=-1, epsilon=1e-5, name=None, out=None):
        y = self._out(name or "layernorm", self.shape(x), name=out)
        ins = [x] + ([scale] if scale is not None else []) + ([bias] if bias is not None else [])
        self._node("LayerNormalization", ins, [y], name, axis=int(axis), epsilon=float(epsilon))
        return y

    def _reduce(self, op, x, axes, keepdims, name, out):
        s = list(self.shape(x))
        nd = len(s)
        ax = sorted(a % nd for a in axes)
        shape = [1 if i in ax else d for i, d in enumerate(s)] if keepdims else \
            [d for i, d in enumerate(s) if i not in ax]
        y = self._out(name or op.lower(), shape, name=out)
        self._node(op, [x], [y], name, axes=[int(a) for a in axes], keepdims=int(keepdims))
        return y

    def reducemean(self, x, axes=(-1,), keepdims=1, name=None, out=None):
        return self._reduce("ReduceMean", x, axes, keepdims, name, out)

    def reducesum(self, x, axes=(-1,), keepdims=1, name=None, out=None):
        return self._reduce("ReduceSum", x, axes, keepdims, name, out)

    # -- shape manipulation ------------------------------------------------------
    def flatten(self, x, axis=1, name=None, out=None):
        s = self.shape(x)
        shape = (int(np.prod(s[:axis])), int(np.prod(s[axis:])))
        y = self._out(name or "flatten", shape, name=out)
        self._node("Flatten", [x], [y], name, axis=int(axis))
        return y

    def reshape(self, x, shape, name=None, out=None):
        s = list(shape)
        total = int(np.prod(self.shape(x)))
        if -1 in s:
            i = s.index(-1)
            rest = int(np.prod([d for d in s if d != -1]))
            s[i] = total // rest
        y = self._out(name or "reshape", s, name=out)
        self._node("Reshape", [x], [y], name, shape=[int(d) for d in s])
        return y

    def transpose(self, x, perm=None, name=None, out=None):
        s = self.shape(x)
        perm = list(perm) if perm is not None else list(range(len(s)))[::-1]
        y = self._out(name or "transpose", [s[p] for p in perm], name=out)
        self._node("Transpose", [x], [y], name, perm=[int(p) for p in perm])
        return y

    def concat(self, xs, axis=1, name=None, out=None):
        s = list(self.shape(xs[0]))
        ax = axis % len(s)
        s[ax] = sum(self.shape(x)[ax] for x in xs)
        y = self._out(name or "concat", s, self.g.tensors[xs[0]].dtype, name=out)
        self._node("Concat", list(xs), [y], name, axis=int(axis))
        return y

    def split(self, x, parts, axis=1, name=None):
        s = list(self.shape(x))
        ax = axis % len(s)
        s[ax] //= parts
        ys = [self._out(name or "split", s, self.g.tensors[x].dtype) for _ in range(parts)]
        self._node("Split", [x], ys, name, axis=int(axis))
        return ys
