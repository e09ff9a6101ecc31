"""Programs of nnc_hip_fused_eltwise (include/nnc_hip.h) and the op-by-op
calls each one replaces, shared by the oracle's and the GPU path's tests.

A step is (op, x, y[, lo, hi]): acc = op(x, y), an operand -1 the previous
step's value or an input index."""

from __future__ import annotations

import numpy as np

import caserun

# op name -> (code, nnc_* entry point of the single op, data operands)
EW_OPS = {"ADD": (0, "nnc_add", 2), "SUB": (1, "nnc_sub", 2), "MUL": (2, "nnc_mul", 2), "DIV": (3, "nnc_div", 2),
          "ADD_RELU": (4, "nnc_add_relu", 2), "ADD_SIGMOID": (5, "nnc_add_sigmoid", 2), "RELU": (6, "nnc_relu", 1),
          "SIGMOID": (7, "nnc_sigmoid", 1), "TANH": (8, "nnc_tanh", 1), "CLIP": (9, "nnc_clip", 1)}

# (inputs, steps): the bandwidth chain's two chains at O3, every op, all four
# inputs, the running value on either side and on both, a single input
EW_PROGRAMS = [
    (2, [("SUB", 0, 1), ("TANH", -1, -1)]),
    (3, [("ADD_RELU", 0, 1), ("MUL", -1, 0), ("CLIP", -1, -1, -6.0, 6.0), ("SIGMOID", -1, -1), ("ADD", -1, 2)]),
    (4, [("DIV", 0, 1), ("ADD_SIGMOID", -1, 2), ("SUB", 3, -1), ("RELU", -1, -1), ("MUL", -1, -1),
         ("CLIP", -1, -1, -0.5, 0.75), ("ADD", 2, -1), ("TANH", -1, -1)]),
    (1, [("RELU", 0, 0), ("SIGMOID", -1, -1)]),
    # the library's other compiled chains: x * y + z (a multiply then an add:
    # no contraction into one rounding), (x + y) * z, relu(x * y),
    # sigmoid(x + y) * y
    (3, [("MUL", 0, 1), ("ADD", -1, 2)]),
    (3, [("ADD", 0, 1), ("MUL", -1, 2)]),
    (2, [("MUL", 0, 1), ("RELU", -1, -1)]),
    (2, [("ADD_SIGMOID", 0, 1), ("MUL", -1, 1)]),
]

# programs with a kernel compiled for them in the library (the rest run on
# the general kernel)
EW_SPECIALIZED = [0, 1, 4, 5, 6, 7]


def ew_arrays(n_in: int, n: int, seed: int) -> list[np.ndarray]:
    """Inputs with exact zeros and values on both sides of the clip bounds;
    the third input of the four-input program is kept away from zero (it
    divides)."""
    rng = np.random.default_rng(seed)
    xs = []
    for i in range(n_in):
        x = (rng.standard_normal(n) * 4).astype(np.float32)
        x[::17] = 0.0
        if i == 1:
            x = np.where(np.abs(x) < 0.25, np.float32(0.5), x).astype(np.float32)
        xs.append(x)
    return xs


def ew_case(n_in: int, steps, arrays, out_key: str = "out") -> dict:
    """nnc_hip_fused_eltwise case over inputs i0..i{n_in-1}; out_key may name
    an input (the output written over it)."""
    prog, consts = [], []
    for st in steps:
        code = EW_OPS[st[0]][0]
        prog += [code, st[1], st[2]]
        consts += [st[3], st[4]] if len(st) > 3 else [0.0, 0.0]
    tensors = {f"i{k}": a for k, a in enumerate(arrays)}
    if out_key not in tensors:
        tensors[out_key] = np.zeros_like(arrays[0])
    return {"name": "ew", "op": "nnc_hip_fused_eltwise", "tensors": tensors,
            "args": [("tl", [f"i{k}" for k in range(n_in)]), ("i", n_in), ("i32", prog), ("i", len(steps)),
                     ("f32", consts), ("t", out_key)], "outputs": [out_key]}


def ew_compose(lib, abi, steps, arrays, mem=None) -> np.ndarray:
    """The program as single nnc_* calls through temporaries."""
    acc = None
    for st in steps:
        _, entry, arity = EW_OPS[st[0]]
        ops = [acc if k < 0 else arrays[k] for k in st[1:1 + arity]]
        tensors = {f"a{j}": v for j, v in enumerate(ops)}
        tensors["o"] = np.zeros_like(arrays[0])
        args = [("t", f"a{j}") for j in range(arity)] + [("t", "o")]
        if st[0] == "CLIP":
            args += [("f", st[3]), ("f", st[4])]
        acc = caserun.run_case(lib, {"name": entry, "op": entry, "tensors": tensors, "args": args,
                                     "outputs": ["o"]}, abi, mem)["o"]
    return acc
