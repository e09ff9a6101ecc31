"""Lowering of graph nodes to nnc_* calls.

Each node becomes one Call: the nnc_* entry point and its argument list,
chosen with the reference code generator's rules (codegen/c_emitter.py:
157-1014): attribute defaults, top/left pads, conv entry-point selection by
kernel kind, Gemm_nt for prepacked constant weights, GlobalAveragePool as an
H x W average pool, Clip bounds from attributes or constant inputs.

Argument specs:
  ("t", name)              Tensor* of a graph tensor
  ("tv", name, shape)      Tensor* viewing that tensor's storage with `shape`
  ("null",)                NULL pointer
  ("i", v) / ("f", v)      int / float
  ("tl", [names])          Tensor** array
  ("i64", [values])        const int64_t* array
  ("i64null",)             NULL int64_t*
  ("i32", [values])        const int* array
  ("f32", [values])        const float* array

DIVERGES from the reference for ReduceMean/ReduceSum over several axes: the
reference passes axes[0] only (c_emitter.py:593-607) and then writes outside
the output. Contiguous axes are merged here into one axis of a view of the
input, so the reduction covers all requested axes.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from .ir import Graph, Node

F32_MAX = 3.402823e38


@dataclass
class Call:
    op: str
    args: list
    node: str = ""


def _t(name):
    return ("t", name)


def _opt(node, idx):
    return _t(node.inputs[idx]) if len(node.inputs) > idx and node.inputs[idx] else ("null",)


def _conv_call(g: Graph, node: Node) -> Call:
    x, w = node.inputs[0], node.inputs[1]
    kh, kw = node.attrs.get("kernel_shape", g.tensors[w].shape[2:4])
    sh, sw = (list(node.attrs.get("strides", [1, 1])) + [1])[:2]
    pads = list(node.attrs.get("pads", [0, 0, 0, 0]))
    ph, pw = (pads + [0, 0])[:2]
    if node.metadata.get("lowering", {}).get("weight_pack") == "tap_major":
        act = {"FusedConvRelu": 1, "FusedConvAddRelu": 1, "FusedConvSigmoid": 2}.get(node.op_type, 0)
        res = _t(node.inputs[3]) if node.op_type == "FusedConvAddRelu" else ("null",)
        return Call("nnc_hip_conv_packed", [_t(x), _t(w), _opt(node, 2), res, _t(node.outputs[0])]
                    + [("i", v) for v in (kh, kw, sh, sw, ph, pw, act)], node.name)
    if node.op_type == "FusedConvAddRelu":
        return Call("nnc_hip_conv_add_relu", [_t(x), _t(w), _opt(node, 2), _t(node.inputs[3]),
                                              _t(node.outputs[0])] + [("i", v) for v in (kh, kw, sh, sw, ph, pw)],
                    node.name)
    io = [_t(x), _t(w), _opt(node, 2), _t(node.outputs[0])]
    if node.op_type == "FusedConvSigmoid":
        return Call("nnc_conv_sigmoid", io + [("i", v) for v in (kh, kw, sh, sw, ph, pw)], node.name)
    prefix = "nnc_conv_relu" if node.op_type == "FusedConvRelu" else "nnc_conv"
    kind = node.metadata.get("lowering", {}).get("kernel_kind")
    if kind == "pointwise_1x1":
        return Call(prefix + "1x1", io + [("i", v) for v in (sh, sw, ph, pw)], node.name)
    if kind == "spatial_3x3":
        return Call(prefix + "3x3_s1", io, node.name)
    if kind == "stem_7x7_s2":
        return Call(prefix + "7x7_s2", io, node.name)
    return Call(prefix, io + [("i", v) for v in (kh, kw, sh, sw, ph, pw)], node.name)


def _pool_args(node):
    k = list(node.attrs.get("kernel_shape", [2, 2]))
    s = list(node.attrs.get("strides", [2, 2]))
    p = list(node.attrs.get("pads", [0, 0, 0, 0]))
    k = k if len(k) >= 2 else [2, 2]
    s = s if len(s) >= 2 else [2, 2]
    p = p if len(p) >= 2 else [0, 0]
    return [("i", k[0]), ("i", k[1]), ("i", s[0]), ("i", s[1]), ("i", p[0]), ("i", p[1])]


def _scalar_const(g: Graph, name: str | None):
    if not name or name not in g.tensors or not g.tensors[name].is_constant:
        return None
    return float(np.asarray(g.tensors[name].data).reshape(-1)[0])


def clip_bounds(g: Graph, node: Node) -> tuple[float, float]:
    """Clip's bounds as the reference code generator takes them
    (c_emitter.py:657-698): attributes, else constant second / third inputs,
    else +-3.402823e38."""
    ins = node.inputs
    lo = node.attrs.get("min", _scalar_const(g, ins[1] if len(ins) > 1 else None))
    hi = node.attrs.get("max", _scalar_const(g, ins[2] if len(ins) > 2 else None))
    lo = -F32_MAX if lo is None or lo == -np.inf else float(lo)
    hi = F32_MAX if hi is None or hi == np.inf else float(hi)
    return lo, hi


def _reduce_call(g: Graph, node: Node, entry: str) -> Call:
    x, y = node.inputs[0], node.outputs[0]
    shape = list(g.tensors[x].shape)
    nd = len(shape)
    axes = node.attrs.get("axes", node.attrs.get("axis", [-1]))
    if not isinstance(axes, (list, tuple)):
        axes = [axes]
    if len(node.inputs) > 1 and node.inputs[1] in g.tensors and g.tensors[node.inputs[1]].is_constant:
        axes = [int(v) for v in np.asarray(g.tensors[node.inputs[1]].data).reshape(-1)]
    keep = int(node.attrs.get("keepdims", 1))
    ax = sorted(a % nd for a in axes)
    if ax != list(range(ax[0], ax[-1] + 1)):
        raise NotImplementedError(f"{node.name}: non-contiguous reduction axes {axes}")
    if len(ax) == 1:
        return Call(entry, [_t(x), _t(y), ("i", ax[0]), ("i", keep)], node.name)
    merged = shape[:ax[0]] + [int(np.prod(shape[ax[0]:ax[-1] + 1]))] + shape[ax[-1] + 1:]
    return Call(entry, [("tv", x, tuple(merged)), _t(y), ("i", ax[0]), ("i", keep)], node.name)


_GENERIC = {
    "Relu": "nnc_relu", "Sigmoid": "nnc_sigmoid", "Tanh": "nnc_tanh", "Sqrt": "nnc_sqrt",
    "Exp": "nnc_exp", "Log": "nnc_log", "Abs": "nnc_abs", "Neg": "nnc_neg",
    "Add": "nnc_add", "Sub": "nnc_sub", "Mul": "nnc_mul", "Div": "nnc_div",
    "Equal": "nnc_equal", "And": "nnc_and", "Greater": "nnc_greater", "Or": "nnc_or",
    "Not": "nnc_not", "Identity": "nnc_identity", "MatMul": "nnc_matmul",
    "FusedAddRelu": "nnc_add_relu", "FusedAddSigmoid": "nnc_add_sigmoid",
}

_CAST = {"float32": 0, "float16": 1, "int32": 2, "int8": 3, "uint8": 4, "bool": 5, "int64": 6}


def _matmul_bias_call(g: Graph, node: Node) -> Call:
    a, w, bias = node.inputs
    out = node.outputs[0]
    if node.op_type == "FusedMatMulBiasRelu":
        return Call("nnc_matmul_relu", [_t(a), _t(w), _t(bias), _t(out)], node.name)
    sa = g.tensors[a].shape
    m = int(np.prod(sa[:-1]))
    n, k = g.tensors[w].shape  # packed [N, K]
    return Call("nnc_gemm_nt", [("tv", a, (m, k)), _t(w), _t(bias), ("tv", out, (m, n)), ("f", 1.0), ("f", 1.0)],
                node.name)


def lower_node(g: Graph, node: Node) -> Call:
    op = node.op_type
    ins, outs = node.inputs, node.outputs
    if op in ("Conv", "FusedConvRelu", "FusedConvSigmoid", "FusedConvAddRelu"):
        return _conv_call(g, node)
    if op == "FusedConvProjRelu":  # 3x3 conv + folded 1x1 projection (include/nnc_hip.h)
        kh, kw = node.attrs.get("kernel_shape", [3, 3])
        sh, sw = (list(node.attrs.get("strides", [1, 1])) + [1])[:2]
        ph, pw = (list(node.attrs.get("pads", [0, 0, 0, 0])) + [0, 0])[:2]
        psh, psw = (list(node.attrs.get("proj_strides", [1, 1])) + [1])[:2]
        return Call("nnc_hip_conv_proj", [_t(ins[0]), _t(ins[1]), _opt(node, 2), _t(ins[3]), _t(outs[0])]
                    + [("i", int(v)) for v in (kh, kw, sh, sw, ph, pw, psh, psw, 1)], node.name)
    if op in ("Spill", "Reload"):  # arena <-> spill pool (include/nnc_hip.h)
        return Call("nnc_hip_transfer", [_t(ins[0]), _t(outs[0])], node.name)
    if op in ("FusedMatMulBias", "FusedMatMulBiasRelu"):
        return _matmul_bias_call(g, node)
    if op == "Gemm":
        args = [_t(ins[0]), _t(ins[1]), _opt(node, 2), _t(outs[0]),
                ("f", float(node.attrs.get("alpha", 1.0))), ("f", float(node.attrs.get("beta", 1.0)))]
        ta, tb = int(node.attrs.get("transA", 0)), int(node.attrs.get("transB", 0))
        if node.metadata.get("lowering", {}).get("weight_pack") == "rhs_transposed_constant" and ta == 0 and tb == 1:
            return Call("nnc_gemm_nt", args, node.name)
        return Call("nnc_gemm", args + [("i", ta), ("i", tb)], node.name)
    if op == "FusedConvMaxPool":  # stem conv + relu streamed into its max pool (include/nnc_hip.h)
        kh, kw = node.attrs.get("kernel_shape", [7, 7])
        sh, sw = (list(node.attrs.get("strides", [1, 1])) + [1])[:2]
        ph, pw = (list(node.attrs.get("pads", [0, 0, 0, 0])) + [0, 0])[:2]
        return Call("nnc_hip_conv_maxpool", [_t(ins[0]), _t(ins[1]), _opt(node, 2), _t(outs[0])]
                    + [("i", int(v)) for v in (kh, kw, sh, sw, ph, pw)], node.name)
    if op == "FusedGapGemm":  # GAP streamed into the classifier (include/nnc_hip.h)
        return Call("nnc_hip_gap_gemm_nt", [_t(ins[0]), _t(ins[1]), _opt(node, 2), _t(outs[0]),
                                            ("f", float(node.attrs.get("alpha", 1.0))),
                                            ("f", float(node.attrs.get("beta", 1.0)))], node.name)
    if op == "FusedAddLayerNorm":  # residual add + layernorm in one pass (include/nnc_hip.h)
        return Call("nnc_hip_add_layernorm", [_t(ins[0]), _t(ins[1]), _opt(node, 2), _opt(node, 3), _t(outs[0]),
                                              ("i", int(node.attrs.get("axis", -1))),
                                              ("f", float(node.attrs.get("epsilon", 1e-5)))], node.name)
    if op == "SliceTranspose":  # a Split piece's reshape + transpose in one copy (include/nnc_hip.h)
        perm = [int(v) for v in node.attrs["perm"]]
        return Call("nnc_hip_transpose_slice", [_t(ins[0]), _t(outs[0]), ("i64", perm), ("i", len(perm)),
                                                ("i", int(node.attrs["col0"])), ("i", int(node.attrs["width"]))],
                    node.name)
    if op == "Attention":  # a transformer layer's attention block in one kernel (include/nnc_hip.h)
        a = node.attrs
        return Call("nnc_hip_attention", [_t(ins[0]), _t(ins[1]), _t(outs[0])]
                    + [("i", int(a[k])) for k in ("batch", "seq", "heads", "head_dim", "q_col", "k_col", "v_col")],
                    node.name)
    if op == "ScaledSoftmax":  # Div by one element + softmax in one pass (include/nnc_hip.h)
        return Call("nnc_hip_scaled_softmax", [_t(ins[0]), _t(ins[1]), _t(outs[0]),
                                               ("i", int(node.attrs.get("axis", -1)))], node.name)
    if op == "FusedEltwise":  # an element-wise chain in one pass (include/nnc_hip.h)
        steps = node.attrs["steps"]
        prog = [v for st in steps for v in (st[0], st[1], st[2])]
        consts = [v for st in steps for v in (st[3], st[4])]
        return Call("nnc_hip_fused_eltwise", [("tl", list(ins)), ("i", len(ins)), ("i32", prog), ("i", len(steps)),
                                              ("f32", consts), _t(outs[0])], node.name)
    if op == "FusedMatMulRelu":
        return Call("nnc_matmul_relu", [_t(ins[0]), _t(ins[1]), _opt(node, 2), _t(outs[0])], node.name)
    if op == "MaxPool":
        return Call("nnc_maxpool2d", [_t(ins[0]), _t(outs[0])] + _pool_args(node), node.name)
    if op == "AveragePool":
        return Call("nnc_avgpool2d", [_t(ins[0]), _t(outs[0])] + _pool_args(node), node.name)
    if op == "GlobalAveragePool":
        h, w = g.tensors[ins[0]].shape[2:4]
        return Call("nnc_avgpool2d", [_t(ins[0]), _t(outs[0]), ("i", h), ("i", w), ("i", h), ("i", w),
                                      ("i", 0), ("i", 0)], node.name)
    if op == "LayerNormalization":
        return Call("nnc_layernorm", [_t(ins[0]), _opt(node, 1), _opt(node, 2), _t(outs[0]),
                                      ("i", int(node.attrs.get("axis", -1))),
                                      ("f", float(node.attrs.get("epsilon", 1e-5)))], node.name)
    if op == "Softmax":
        return Call("nnc_softmax", [_t(ins[0]), _t(outs[0]), ("i", int(node.attrs.get("axis", -1)))], node.name)
    if op in ("ReduceMean", "ReduceSum"):
        return _reduce_call(g, node, "nnc_reducemean" if op == "ReduceMean" else "nnc_reducesum")
    if op == "Flatten":
        return Call("nnc_flatten", [_t(ins[0]), _t(outs[0]), ("i", int(node.attrs.get("axis", 1)))], node.name)
    if op == "Reshape":
        shape = node.attrs.get("shape") or list(g.tensors[outs[0]].shape)
        return Call("nnc_reshape", [_t(ins[0]), _t(outs[0]), ("i64", list(shape)), ("i", len(shape))], node.name)
    if op == "Transpose":
        perm = node.attrs.get("perm")
        nd = len(g.tensors[ins[0]].shape)
        pa = ("i64", list(perm)) if perm else ("i64null",)
        return Call("nnc_transpose", [_t(ins[0]), _t(outs[0]), pa, ("i", nd)], node.name)
    if op == "Squeeze":
        return Call("nnc_squeeze", [_t(ins[0]), _t(outs[0]), ("i", int(node.attrs.get("axis", 0)))], node.name)
    if op == "Unsqueeze":
        return Call("nnc_unsqueeze", [_t(ins[0]), _t(outs[0]), ("i", int(node.attrs.get("axis", 0)))], node.name)
    if op == "Concat":
        return Call("nnc_concat", [("tl", list(ins)), _t(outs[0]), ("i", len(ins)),
                                   ("i", int(node.attrs.get("axis", 0)))], node.name)
    if op == "Split":
        return Call("nnc_split", [_t(ins[0]), ("tl", list(outs)), ("i", len(outs)),
                                  ("i", int(node.attrs.get("axis", 0)))], node.name)
    if op == "Clip":
        lo, hi = clip_bounds(g, node)
        return Call("nnc_clip", [_t(ins[0]), _t(outs[0]), ("f", lo), ("f", hi)], node.name)
    if op == "Pow":  # always x*x in the reference runtime (ops.c:2449-2461)
        return Call("nnc_pow", [_t(ins[0]), _t(outs[0])], node.name)
    if op == "Tile":
        rep = ins[1] if len(ins) > 1 else None
        if rep and g.tensors[rep].is_constant:
            vals = [int(v) for v in np.asarray(g.tensors[rep].data).reshape(-1)]
            return Call("nnc_tile", [_t(ins[0]), _t(outs[0]), ("i64", vals), ("i", len(vals))], node.name)
        return Call("nnc_tile", [_t(ins[0]), _t(outs[0]), ("i64null",), ("i", len(g.tensors[outs[0]].shape))],
                    node.name)
    if op == "Shape":
        dims = list(g.tensors[ins[0]].shape)
        return Call("nnc_shape", [_t(ins[0]), _t(outs[0]), ("i64", dims), ("i", len(dims))], node.name)
    if op == "ConstantOfShape":
        return Call("nnc_constantofshape", [_t(outs[0]), ("f", float(node.attrs.get("value", 0.0))),
                                            ("i", len(g.tensors[outs[0]].shape))], node.name)
    if op == "Expand":
        nd = len(g.tensors[outs[0]].shape)
        return Call("nnc_expand", [_t(ins[0]), _t(outs[0]), ("i64", list(g.tensors[outs[0]].shape)), ("i", nd)],
                    node.name)
    if op == "Cast":
        to = node.attrs.get("to", "float32")
        return Call("nnc_cast", [_t(ins[0]), _t(outs[0]), ("i", _CAST.get(to, 0) if isinstance(to, str) else int(to))],
                    node.name)
    if op == "Gather":
        dd = 1 if g.tensors[ins[0]].dtype == "int64" else 0
        return Call("nnc_gather", [_t(ins[0]), _t(ins[1]), _t(outs[0]), ("i", int(node.attrs.get("axis", 0))),
                                   ("i", dd)], node.name)
    if op == "LSTM":
        direction = {"forward": 0, "reverse": 1, "bidirectional": 2}.get(node.attrs.get("direction", "forward"), 0)
        args = [_t(ins[0]), _t(ins[1]), _t(ins[2]), _opt(node, 3)] + [_t(o) for o in outs[:3]]
        return Call("nnc_lstm", args + [("i", direction), ("i", int(node.attrs.get("hidden_size", 0)))], node.name)
    if op == "BatchNormalization":
        raise NotImplementedError(f"{node.name}: BatchNormalization must be folded into the "
                                  "preceding Conv (the reference runtime's batchnorm is a no-op)")
    if op in _GENERIC:
        return Call(_GENERIC[op], [_t(i) for i in ins] + [_t(o) for o in outs], node.name)
    raise NotImplementedError(f"no nnc_* lowering for op {op!r} ({node.name})")


def lower(g: Graph, order: list[Node], aliases: dict[str, str] | None = None) -> list[Call]:
    """One call per node, except view ops the plan turned into aliases."""
    aliases = aliases or {}
    return [lower_node(g, n) for n in order if not (n.outputs and n.outputs[0] in aliases)]
