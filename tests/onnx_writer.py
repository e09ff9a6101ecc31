"""A minimal ONNX protobuf encoder for the tests (the onnx package is not
installed): writes a GraphBuilder graph, or hand-made nodes, as a ModelProto
with the field numbers of onnx.proto (proto2: repeated scalars unpacked),
so that compiler/onnx_reader.py is exercised on real wire-format files."""

from __future__ import annotations

import struct

import numpy as np

_ELEM = {"float32": 1, "uint8": 2, "int8": 3, "int32": 6, "int64": 7, "bool": 9, "float16": 10, "float64": 11}


def _varint(v: int) -> bytes:
    v &= (1 << 64) - 1
    out = bytearray()
    while True:
        b = v & 0x7F
        v >>= 7
        if v:
            out.append(b | 0x80)
        else:
            out.append(b)
            return bytes(out)


def _key(num: int, wt: int) -> bytes:
    return _varint((num << 3) | wt)


def f_varint(num: int, v: int) -> bytes:
    return _key(num, 0) + _varint(v)


def f_bytes(num: int, data: bytes) -> bytes:
    return _key(num, 2) + _varint(len(data)) + data


def f_str(num: int, s: str) -> bytes:
    return f_bytes(num, s.encode())


def f_float(num: int, v: float) -> bytes:
    return _key(num, 5) + struct.pack("<f", v)


def tensor(name: str, arr: np.ndarray) -> bytes:
    arr = np.ascontiguousarray(arr)
    out = b"".join(f_varint(1, d) for d in arr.shape)
    out += f_varint(2, _ELEM[arr.dtype.name]) + f_str(8, name) + f_bytes(9, arr.astype(arr.dtype.newbyteorder("<")).tobytes())
    return out


def attribute(name: str, value) -> bytes:
    out = f_str(1, name)
    if isinstance(value, float):
        return out + f_float(2, value) + f_varint(20, 1)
    if isinstance(value, (bool, int, np.integer)):
        return out + f_varint(3, int(value)) + f_varint(20, 2)
    if isinstance(value, str):
        return out + f_bytes(4, value.encode()) + f_varint(20, 3)
    if isinstance(value, np.ndarray):
        return out + f_bytes(5, tensor("", value)) + f_varint(20, 4)
    vals = list(value)
    if vals and isinstance(vals[0], float):
        return out + b"".join(f_float(7, x) for x in vals) + f_varint(20, 6)
    return out + b"".join(f_varint(8, int(x)) for x in vals) + f_varint(20, 7)


def node(op: str, inputs, outputs, name: str = "", **attrs) -> bytes:
    out = b"".join(f_str(1, i) for i in inputs) + b"".join(f_str(2, o) for o in outputs)
    out += f_str(3, name) + f_str(4, op)
    out += b"".join(f_bytes(5, attribute(k, v)) for k, v in attrs.items())
    return out


def value_info(name: str, shape, dtype: str = "float32") -> bytes:
    dims = b"".join(f_bytes(1, f_varint(1, d)) for d in shape)
    ttype = f_varint(1, _ELEM[dtype]) + f_bytes(2, dims)
    return f_str(1, name) + f_bytes(2, f_bytes(1, ttype))


def model(nodes: list[bytes], inits: dict[str, np.ndarray], inputs, outputs, name: str = "g") -> bytes:
    g = b"".join(f_bytes(1, n) for n in nodes) + f_str(2, name)
    g += b"".join(f_bytes(5, tensor(k, v)) for k, v in inits.items())
    g += b"".join(f_bytes(11, value_info(*i)) for i in inputs)
    g += b"".join(f_bytes(12, value_info(*o)) for o in outputs)
    opset = f_str(1, "") + f_varint(2, 17)
    return f_varint(1, 8) + f_str(2, "nnc-tests") + f_bytes(8, opset) + f_bytes(7, g)


def from_graph(graph) -> bytes:
    """A GraphBuilder graph as an ONNX model (Reshape's shape attribute
    becomes an int64 initializer, as exporters write it)."""
    inits = {k: np.asarray(t.data) for k, t in graph.constants.items()}
    nodes = []
    for n in graph.nodes:
        attrs = dict(n.attrs)
        ins = list(n.inputs)
        if n.op_type == "Reshape":
            shp = f"{n.name}::shape"
            inits[shp] = np.asarray(attrs.pop("shape"), np.int64)
            ins.append(shp)
        nodes.append(node(n.op_type, ins, n.outputs, n.name, **attrs))
    inputs = [(i, graph.tensors[i].shape, graph.tensors[i].dtype) for i in graph.inputs]
    outputs = [(o, graph.tensors[o].shape, graph.tensors[o].dtype) for o in graph.outputs]
    return model(nodes, inits, inputs, outputs, graph.name if hasattr(graph, "name") else "g")
