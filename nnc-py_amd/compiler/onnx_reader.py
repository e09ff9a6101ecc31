"""ONNX model files -> Graph, without the onnx package.

The reference frontend (src/nnc_py/frontend/onnx_loader.py) loads models
with `onnx` and simplifies them with `onnxsim` (constant folding, Conv+BN
fusion). Neither is available offline, so this module decodes the ONNX
protobuf wire format itself (ModelProto / GraphProto / NodeProto /
AttributeProto / TensorProto / ValueInfoProto, the field numbers of
onnx.proto) and builds the graph with GraphBuilder, which infers every
output shape. BatchNormalization after a Conv with constant parameters is
folded into the conv's weight and bias (what onnxsim does for the exported
models); Constant nodes become initializers; Identity/Dropout pass through.

    from nnc_py_amd.compiler.onnx_reader import load_onnx
    graph = load_onnx("resnet18.onnx")
"""

from __future__ import annotations

import struct
from pathlib import Path

import numpy as np

from .builder import GraphBuilder
from .ir import Graph

# TensorProto.DataType -> numpy
_DTYPE = {1: np.float32, 2: np.uint8, 3: np.int8, 5: np.int16, 6: np.int32, 7: np.int64, 9: np.bool_,
          10: np.float16, 11: np.float64}


# ---------------------------------------------------------------------------
# protobuf wire format
# ---------------------------------------------------------------------------
def _varint(buf: bytes, pos: int) -> tuple[int, int]:
    out = shift = 0
    while True:
        b = buf[pos]
        pos += 1
        out |= (b & 0x7F) << shift
        if b < 0x80:
            return out, pos
        shift += 7


def _fields(buf: bytes):
    """(field number, wire type, value) of one message; value is an int for
    varint / fixed types and a bytes slice for length-delimited ones."""
    pos, end = 0, len(buf)
    while pos < end:
        key, pos = _varint(buf, pos)
        num, wt = key >> 3, key & 7
        if wt == 0:
            val, pos = _varint(buf, pos)
        elif wt == 1:
            val = buf[pos:pos + 8]
            pos += 8
        elif wt == 2:
            n, pos = _varint(buf, pos)
            val = buf[pos:pos + n]
            pos += n
        elif wt == 5:
            val = buf[pos:pos + 4]
            pos += 4
        else:
            raise ValueError(f"unsupported protobuf wire type {wt}")
        yield num, wt, val


def _signed(v: int) -> int:
    return v - (1 << 64) if v >= 1 << 63 else v


def _packed_varints(val, wt) -> list[int]:
    if wt == 0:
        return [_signed(val)]
    out, pos = [], 0
    while pos < len(val):
        v, pos = _varint(val, pos)
        out.append(_signed(v))
    return out


def _packed_floats(val, wt) -> list[float]:
    if wt == 5:
        return [struct.unpack("<f", val)[0]]
    return list(struct.unpack(f"<{len(val) // 4}f", val))


def _tensor(buf: bytes) -> tuple[str, np.ndarray]:
    dims, dtype, name, raw = [], 1, "", None
    floats, ints32, ints64, doubles = [], [], [], []
    for num, wt, val in _fields(buf):
        if num == 1:
            dims += _packed_varints(val, wt)
        elif num == 2:
            dtype = val
        elif num == 4:
            floats += _packed_floats(val, wt)
        elif num == 5:
            ints32 += _packed_varints(val, wt)
        elif num == 7:
            ints64 += _packed_varints(val, wt)
        elif num == 8:
            name = bytes(val).decode()
        elif num == 9:
            raw = bytes(val)
        elif num == 10:
            doubles += list(struct.unpack(f"<{len(val) // 8}d", val)) if wt == 2 else [struct.unpack("<d", val)[0]]
        elif num == 14 and val == 1:
            raise ValueError(f"tensor {name!r}: external data is not supported")
    np_dtype = _DTYPE.get(dtype)
    if np_dtype is None:
        raise ValueError(f"tensor {name!r}: unsupported data type {dtype}")
    if raw is not None:
        arr = np.frombuffer(raw, dtype=np.dtype(np_dtype).newbyteorder("<")).astype(np_dtype)
    elif floats:
        arr = np.array(floats, dtype=np_dtype)
    elif ints64:
        arr = np.array(ints64, dtype=np_dtype)
    elif ints32:
        arr = np.array(ints32, dtype=np_dtype)
    elif doubles:
        arr = np.array(doubles, dtype=np_dtype)
    else:
        arr = np.zeros(0, dtype=np_dtype)
    return name, arr.reshape(dims) if dims else arr.reshape(())


def _attribute(buf: bytes):
    name, value = "", None
    floats, ints, strings = [], [], []
    for num, wt, val in _fields(buf):
        if num == 1:
            name = bytes(val).decode()
        elif num == 2:
            value = struct.unpack("<f", val)[0]
        elif num == 3:
            value = _signed(val)
        elif num == 4:
            value = bytes(val).decode(errors="replace")
        elif num == 5:
            value = _tensor(val)[1]
        elif num == 7:
            floats += _packed_floats(val, wt)
        elif num == 8:
            ints += _packed_varints(val, wt)
        elif num == 9:
            strings.append(bytes(val).decode(errors="replace"))
    if value is None:
        value = ints if ints else floats if floats else strings if strings else None
    return name, value


def _value_info(buf: bytes) -> tuple[str, list | None, int]:
    name, shape, elem = "", None, 1
    for num, _, val in _fields(buf):
        if num == 1:
            name = bytes(val).decode()
        elif num == 2:
            for tnum, _, tval in _fields(val):
                if tnum != 1:
                    continue
                for snum, _, sval in _fields(tval):
                    if snum == 1:
                        elem = sval
                    elif snum == 2:
                        shape = []
                        for dnum, _, dval in _fields(sval):
                            if dnum != 1:
                                continue
                            dim = None
                            for fnum, _, fval in _fields(dval):
                                if fnum == 1:
                                    dim = _signed(fval)
                            shape.append(dim)
    return name, shape, elem


def _parse(data: bytes):
    graph_buf = None
    for num, _, val in _fields(data):
        if num == 7:
            graph_buf = val
    if graph_buf is None:
        raise ValueError("not an ONNX model: no graph")
    nodes, inits, inputs, outputs, name = [], {}, [], [], "model"
    for num, _, val in _fields(graph_buf):
        if num == 1:
            node = {"inputs": [], "outputs": [], "name": "", "op": "", "attrs": {}}
            for nnum, _, nval in _fields(val):
                if nnum == 1:
                    node["inputs"].append(bytes(nval).decode())
                elif nnum == 2:
                    node["outputs"].append(bytes(nval).decode())
                elif nnum == 3:
                    node["name"] = bytes(nval).decode()
                elif nnum == 4:
                    node["op"] = bytes(nval).decode()
                elif nnum == 5:
                    k, v = _attribute(nval)
                    node["attrs"][k] = v
            nodes.append(node)
        elif num == 2:
            name = bytes(val).decode()
        elif num == 5:
            k, arr = _tensor(val)
            inits[k] = arr
        elif num == 11:
            inputs.append(_value_info(val))
        elif num == 12:
            outputs.append(_value_info(val))
    return name, nodes, inits, inputs, outputs


# ---------------------------------------------------------------------------
# ONNX nodes -> GraphBuilder
# ---------------------------------------------------------------------------
def load_onnx(path: str | Path, input_shapes: dict[str, tuple] | None = None) -> Graph:
    """Graph of an .onnx file. Symbolic input dimensions need `input_shapes`
    (the reference requires static shapes too)."""
    name, nodes, inits, inputs, outputs = _parse(Path(path).read_bytes())
    b = GraphBuilder(name or "model")
    values: dict[str, str] = {}
    consts: dict[str, np.ndarray] = {}

    def const(nm: str, arr: np.ndarray) -> str:
        arr = np.asarray(arr)
        if arr.dtype == np.float64:
            arr = arr.astype(np.float32)
        consts[nm] = arr
        values[nm] = b.const(nm, arr)
        return values[nm]

    for k, arr in inits.items():
        const(k, arr)
    for nm, shape, elem in inputs:
        if nm in values:
            continue  # an initializer also listed as graph input
        shp = (input_shapes or {}).get(nm, shape)
        if shp is None or any(d is None or d <= 0 for d in shp):
            raise ValueError(f"input {nm!r} has a symbolic shape {shape}; pass input_shapes")
        values[nm] = b.input(nm, tuple(int(d) for d in shp), np.dtype(_DTYPE.get(elem, np.float32)).name)

    def v(nm):
        return values[nm] if nm else None

    # BatchNormalization folding needs the conv that feeds it: remember producers
    producer = {}
    for n in nodes:
        for o in n["outputs"]:
            producer[o] = n
    folded: dict[str, tuple] = {}  # conv output name -> (scale, shift) to apply
    for n in nodes:
        if n["op"] != "BatchNormalization":
            continue
        x = n["inputs"][0]
        p = producer.get(x)
        if p and p["op"] == "Conv" and all(i in consts or i in inits for i in n["inputs"][1:5]) and \
                sum(1 for m in nodes if x in m["inputs"]) == 1:
            g_, b_, m_, var = (np.asarray(inits.get(i, consts.get(i)), np.float64) for i in n["inputs"][1:5])
            eps = float(n["attrs"].get("epsilon", 1e-5))
            scale = g_ / np.sqrt(var + eps)
            folded[x] = (scale, b_ - m_ * scale, n["outputs"][0])

    for n in nodes:
        op, ins, outs, at, nm = n["op"], n["inputs"], n["outputs"], n["attrs"], n["name"] or None
        if op == "BatchNormalization" and ins[0] in folded:
            continue  # folded into the conv, which produced outs[0]
        if op == "Constant":
            val = at.get("value")
            if val is None:
                val = at.get("value_float", at.get("value_int", at.get("value_floats", at.get("value_ints"))))
            const(outs[0], np.asarray(val))
            continue
        if op in ("Identity", "Dropout"):
            values[outs[0]] = values[ins[0]]
            continue
        out = outs[0] if outs else None
        if op == "Conv":
            if int(at.get("group", 1)) != 1:
                raise NotImplementedError(f"{nm}: grouped convolution")
            wname = values[ins[1]]
            bname = values[ins[2]] if len(ins) > 2 and ins[2] else None
            if out in folded:
                # Conv followed by BatchNormalization: scale the weights and
                # shift the bias per output channel
                scale, shift, bn_out = folded[out]
                w = consts[ins[1]].astype(np.float64) * scale.reshape(-1, 1, 1, 1)
                bias = consts[ins[2]].astype(np.float64) if bname else np.zeros(w.shape[0])
                wname = const(f"{bn_out}::weight", w.astype(np.float32))
                bname = const(f"{bn_out}::bias", (bias * scale + shift).astype(np.float32))
                out = bn_out
            pads = tuple(at.get("pads", [0, 0, 0, 0]))
            values[out] = b.conv(values[ins[0]], wname, bname, strides=tuple(at.get("strides", [1, 1])),
                                 pads=pads, name=nm, out=out)
            continue
        if op in ("Relu", "Sigmoid", "Tanh", "Sqrt", "Exp"):
            values[out] = getattr(b, op.lower())(values[ins[0]], name=nm, out=out)
        elif op in ("Add", "Sub", "Mul", "Div"):
            values[out] = getattr(b, op.lower())(values[ins[0]], values[ins[1]], name=nm, out=out)
        elif op == "MaxPool" or op == "AveragePool":
            k = tuple(at.get("kernel_shape", [2, 2]))
            s = tuple(at.get("strides", [1, 1]))
            p = tuple(at.get("pads", [0, 0, 0, 0]))
            fn = b.maxpool if op == "MaxPool" else b.avgpool
            values[out] = fn(values[ins[0]], k, s, p, name=nm, out=out)
        elif op == "GlobalAveragePool":
            values[out] = b.global_avgpool(values[ins[0]], name=nm, out=out)
        elif op == "Gemm":
            values[out] = b.gemm(values[ins[0]], values[ins[1]], v(ins[2]) if len(ins) > 2 else None,
                                 alpha=at.get("alpha", 1.0), beta=at.get("beta", 1.0),
                                 transA=at.get("transA", 0), transB=at.get("transB", 0), name=nm, out=out)
        elif op == "MatMul":
            values[out] = b.matmul(values[ins[0]], values[ins[1]], name=nm, out=out)
        elif op == "Flatten":
            values[out] = b.flatten(values[ins[0]], int(at.get("axis", 1)), name=nm, out=out)
        elif op == "Reshape":
            shape = at.get("shape")
            if shape is None:
                shape = [int(d) for d in consts[ins[1]].reshape(-1)]
            src = b.shape(values[ins[0]])
            shape = [src[i] if d == 0 else d for i, d in enumerate(shape)]
            values[out] = b.reshape(values[ins[0]], shape, name=nm, out=out)
        elif op == "Transpose":
            values[out] = b.transpose(values[ins[0]], at.get("perm"), name=nm, out=out)
        elif op == "Concat":
            values[out] = b.concat([values[i] for i in ins], int(at.get("axis", 0)), name=nm, out=out)
        elif op == "Split":
            ys = b.split(values[ins[0]], len(outs), int(at.get("axis", 0)), name=nm)
            for o, y in zip(outs, ys):
                values[o] = y
        elif op == "Softmax":
            values[out] = b.softmax(values[ins[0]], int(at.get("axis", -1)), name=nm, out=out)
        elif op == "LayerNormalization":
            values[out] = b.layernorm(values[ins[0]], v(ins[1]) if len(ins) > 1 else None,
                                      v(ins[2]) if len(ins) > 2 else None, int(at.get("axis", -1)),
                                      float(at.get("epsilon", 1e-5)), name=nm, out=out)
        elif op in ("ReduceMean", "ReduceSum"):
            axes = at.get("axes")
            if axes is None and len(ins) > 1 and ins[1]:
                axes = [int(d) for d in consts[ins[1]].reshape(-1)]
            fn = b.reducemean if op == "ReduceMean" else b.reducesum
            values[out] = fn(values[ins[0]], tuple(axes if axes is not None else [-1]),
                             int(at.get("keepdims", 1)), name=nm, out=out)
        elif op == "Clip":
            lo = at.get("min", float(consts[ins[1]]) if len(ins) > 1 and ins[1] else None)
            hi = at.get("max", float(consts[ins[2]]) if len(ins) > 2 and ins[2] else None)
            values[out] = b.clip(values[ins[0]], lo, hi, name=nm, out=out)
        elif op == "BatchNormalization":
            raise NotImplementedError(f"{nm}: BatchNormalization that does not follow a Conv with constant "
                                      "parameters cannot be folded (the reference runtime's batchnorm is a no-op)")
        else:
            raise NotImplementedError(f"ONNX op {op!r} ({nm}) is not supported by this frontend")
    for nm, _, _ in outputs:
        b.output(values[nm])
    return b.build()
