"""Catalogue of nnc_* calls used as golden vectors.

Each builder returns a case dict in the format of tests/caserun.py. Inputs are
seeded (numpy default_rng, seed per case) or literal. Literal cases replay the
reference's own known-answer tests (tests/test_x86_runtime.py and
tests/test_numerical_accuracy.py of the reference, cited per case).

`hip` marks cases whose libnnc_hip result is checked differently from the
reference output, with the reason:
  "batched"   reference batched MatMul steps by batch count (ops.c:1687-1704);
              the HIP kernel implements MatMul semantics, compared with the
              oracle's 2-D path per batch.
  "skip"      argument combination the reference accepts but that is
              undefined (reads or writes outside a buffer) and that the HIP
              library rejects; the test checks the rejection instead.
"""

from __future__ import annotations

import numpy as np

F32 = np.float32


def _rng(seed):
    return np.random.default_rng(seed)


def _normal(rng, shape, scale=1.0):
    return (rng.standard_normal(shape) * scale).astype(F32)


def conv_out_hw(h, w, kh, kw, sh, sw, ph, pw):
    return (h + 2 * ph - kh) // sh + 1, (w + 2 * pw - kw) // sw + 1


def case(name, op, tensors, args, outputs, bar="exact", **extra):
    d = dict(name=name, op=op, tensors=tensors, args=args, outputs=outputs, bar=bar)
    d.update(extra)
    return d


# --------------------------------------------------------------------------
# element-wise
# --------------------------------------------------------------------------
def binary_cases():
    out = []
    ops = ["nnc_add", "nnc_sub", "nnc_mul", "nnc_div", "nnc_add_relu", "nnc_add_sigmoid"]
    shapes = [
        ("same", (2, 3, 4, 5), (2, 3, 4, 5), (2, 3, 4, 5)),
        ("bscalar", (2, 3, 4, 5), (1,), (2, 3, 4, 5)),
        ("ascalar", (1,), (3, 7), (3, 7)),
        ("btrail", (4, 6), (6,), (4, 6)),
        ("atrail", (6,), (4, 6), (4, 6)),
        ("keepdims", (1, 4, 8), (1, 4, 1), (1, 4, 8)),  # flat-modulo, not numpy
        ("both_small", (6,), (4,), (12,)),              # only min() written
        ("odd", (1037,), (1037,), (1037,)),
    ]
    seed = 100
    for op in ops:
        for tag, sa, sb, so in shapes:
            rng = _rng(seed)
            seed += 1
            a = _normal(rng, sa)
            b = _normal(rng, sb)
            if op == "nnc_div":
                b = np.where(np.abs(b) < 0.1, F32(0.5), b).astype(F32)
            o = np.full(so, 7.0, F32)  # sentinel shows unwritten elements
            bar = "exact" if op in ("nnc_add", "nnc_sub", "nnc_mul", "nnc_div", "nnc_add_relu") else "fp"
            out.append(case(f"{op}_{tag}", op, {"a": a, "b": b, "out": o},
                            [("t", "a"), ("t", "b"), ("t", "out")], ["out"], bar))
    # in-place aliasing (cost_aware reuses a dying input as the output)
    return out


def unary_cases():
    out = []
    rng = _rng(7)
    base = _normal(rng, (3, 5, 7, 11), 3.0)
    base.ravel()[:6] = [0.0, -0.0, 1e-30, -1e-30, 88.0, -90.0]
    pos = np.abs(base) + F32(1e-3)
    specs = [
        ("nnc_relu", base, "exact"),
        ("nnc_sigmoid", base, "fp"),
        ("nnc_tanh", base, "fp"),
        ("nnc_sqrt", base, "fp"),  # negatives -> NaN
        ("nnc_pow", base, "exact"),
        ("nnc_exp", np.clip(base, -80, 80).astype(F32), "fp"),
        ("nnc_log", base, "fp"),   # <= 0 -> NaN
        ("nnc_abs", base, "exact"),
        ("nnc_neg", base, "exact"),
        ("nnc_log", pos, "fp"),
    ]
    for i, (op, x, bar) in enumerate(specs):
        o = np.zeros_like(x)
        out.append(case(f"{op}_{i}", op, {"x": x.copy(), "out": o},
                        [("t", "x"), ("t", "out")], ["out"], bar))
    for lo, hi, tag in [(-6.0, 6.0, "relu6"), (-3.402823e38, 3.402823e38, "default"),
                        (0.0, 1.0, "unit")]:
        o = np.zeros_like(base)
        out.append(case(f"nnc_clip_{tag}", "nnc_clip", {"x": base.copy(), "out": o},
                        [("t", "x"), ("t", "out"), ("f", lo), ("f", hi)], ["out"], "exact"))
    # literal KATs, reference tests/test_x86_runtime.py:536-579, 1593-1670
    lit = {
        "nnc_relu": [[-1.0, 2.0], [-3.0, 4.0]],
        "nnc_sigmoid": [[0.0, 1.0], [-1.0, 2.0]],
        "nnc_tanh": [[0.0, 1.0], [-1.0, 2.0]],
        "nnc_sqrt": [[1.0, 4.0], [9.0, 16.0]],
        "nnc_exp": [[0.0, 1.0], [2.0, 3.0]],
        "nnc_log": [[1.0, 2.0], [3.0, 4.0]],
        "nnc_abs": [[-1.0, -2.0], [3.0, -4.0]],
        "nnc_neg": [[1.0, 2.0], [3.0, 4.0]],
    }
    for op, v in lit.items():
        x = np.array(v, F32)
        out.append(case(f"{op}_kat", op, {"x": x, "out": np.zeros_like(x)},
                        [("t", "x"), ("t", "out")], ["out"],
                        "exact" if op in ("nnc_relu", "nnc_abs", "nnc_neg", "nnc_sqrt") else "fp"))
    return out


def logic_cases():
    out = []
    # reference tests/test_x86_runtime.py:1523-1591
    a = np.array([[1.0, 2.0], [3.0, 4.0]], F32)
    out.append(case("nnc_equal_kat", "nnc_equal",
                    {"a": a, "b": np.array([[1.0, 2.0], [3.0, 5.0]], F32), "out": np.zeros_like(a)},
                    [("t", "a"), ("t", "b"), ("t", "out")], ["out"]))
    out.append(case("nnc_equal_bcast_kat", "nnc_equal",
                    {"a": a, "b": np.array([1.0, 2.0], F32), "out": np.zeros_like(a)},
                    [("t", "a"), ("t", "b"), ("t", "out")], ["out"]))
    out.append(case("nnc_and_kat", "nnc_and",
                    {"a": np.array([[1.0, 0.0], [1.0, 1.0]], F32),
                     "b": np.array([[1.0, 1.0], [0.0, 1.0]], F32), "out": np.zeros_like(a)},
                    [("t", "a"), ("t", "b"), ("t", "out")], ["out"]))
    out.append(case("nnc_and_bcast_kat", "nnc_and",
                    {"a": np.array([[1.0, 0.0], [0.0, 1.0]], F32),
                     "b": np.array([1.0, 0.0], F32), "out": np.zeros_like(a)},
                    [("t", "a"), ("t", "b"), ("t", "out")], ["out"]))
    rng = _rng(11)
    x = np.round(_normal(rng, (4, 33)) * 2) / 2
    y = np.round(_normal(rng, (4, 33)) * 2) / 2
    out.append(case("nnc_equal_rand", "nnc_equal", {"a": x, "b": y, "out": np.zeros_like(x)},
                    [("t", "a"), ("t", "b"), ("t", "out")], ["out"]))
    out.append(case("nnc_greater_rand", "nnc_greater",
                    {"a": x, "b": y[0].copy(), "out": np.zeros(x.shape, np.uint8)},
                    [("t", "a"), ("t", "b"), ("t", "out")], ["out"]))
    p = (rng.random((5, 13)) > 0.5).astype(np.uint8)
    q = (rng.random((5, 13)) > 0.5).astype(np.uint8)
    out.append(case("nnc_or_rand", "nnc_or", {"a": p, "b": q, "out": np.zeros_like(p)},
                    [("t", "a"), ("t", "b"), ("t", "out")], ["out"]))
    out.append(case("nnc_not_rand", "nnc_not", {"a": p, "out": np.zeros_like(p)},
                    [("t", "a"), ("t", "out")], ["out"]))
    return out


# --------------------------------------------------------------------------
# softmax / layernorm / reductions
# --------------------------------------------------------------------------
def softmax_cases():
    out = []
    # reference tests/test_x86_runtime.py:581-597
    x = np.array([[1.0, 2.0, 3.0], [4.0, 5.0, 6.0]], F32)
    out.append(case("nnc_softmax_kat", "nnc_softmax", {"x": x, "out": np.zeros_like(x)},
                    [("t", "x"), ("t", "out"), ("i", 1)], ["out"], "fp"))
    for i, (shape, axis) in enumerate([((5, 37), -1), ((3, 4, 129), -1), ((2, 5, 3), 1),
                                       ((2, 3, 4, 9), 0), ((4, 1024), 1), ((2, 4, 16, 16), 3)]):
        rng = _rng(200 + i)
        x = _normal(rng, shape, 3.0)
        out.append(case(f"nnc_softmax_{i}", "nnc_softmax", {"x": x, "out": np.zeros_like(x)},
                        [("t", "x"), ("t", "out"), ("i", axis)], ["out"], "fp"))
    return out


def layernorm_cases():
    out = []
    for i, (shape, axis, affine) in enumerate([((6, 33), -1, True), ((4, 768), -1, True),
                                               ((2, 3, 4, 5), 2, True), ((3, 7, 16), -1, False),
                                               ((2, 8, 256), 2, True)]):
        rng = _rng(300 + i)
        x = _normal(rng, shape, 2.0) + F32(0.5)
        d = shape[axis]
        t = {"x": x, "out": np.zeros_like(x)}
        args = [("t", "x")]
        if affine:
            t["g"] = _normal(rng, (d,))
            t["b"] = _normal(rng, (d,))
            args += [("t", "g"), ("t", "b")]
        else:
            args += [("null",), ("null",)]
        args += [("t", "out"), ("i", axis), ("f", 1e-5)]
        out.append(case(f"nnc_layernorm_{i}", "nnc_layernorm", t, args, ["out"], "fp"))
    return out


def reduce_cases():
    out = []
    a = np.array([[1.0, 2.0, 3.0], [4.0, 5.0, 6.0]], F32)
    # reference tests/test_x86_runtime.py:1423-1481
    for op, axis, keep, oshape in [("nnc_reducemean", 1, 1, (2, 1)), ("nnc_reducemean", 1, 0, (2,)),
                                   ("nnc_reducesum", 0, 1, (1, 3)), ("nnc_reducesum", 0, 0, (3,))]:
        out.append(case(f"{op}_kat_a{axis}_k{keep}", op,
                        {"x": a, "out": np.zeros(oshape, F32)},
                        [("t", "x"), ("t", "out"), ("i", axis), ("i", keep)], ["out"], "fp"))
    # Kahan KATs, reference tests/test_numerical_accuracy.py:174-260
    big = np.array([[1e7] + [1.0] * 10000], F32)
    out.append(case("nnc_reducesum_kahan_1e7", "nnc_reducesum",
                    {"x": big, "out": np.zeros((1, 1), F32)},
                    [("t", "x"), ("t", "out"), ("i", 1), ("i", 1)], ["out"], "fp"))
    small = np.array([[1.0 + 1e-7] * 100000], F32)
    out.append(case("nnc_reducesum_kahan_many", "nnc_reducesum",
                    {"x": small, "out": np.zeros((1, 1), F32)},
                    [("t", "x"), ("t", "out"), ("i", 1), ("i", 1)], ["out"], "fp"))
    mean = np.array([[1e5] + [0.1] * 10000], F32)
    out.append(case("nnc_reducemean_kahan", "nnc_reducemean",
                    {"x": mean, "out": np.zeros((1, 1), F32)},
                    [("t", "x"), ("t", "out"), ("i", 1), ("i", 1)], ["out"], "fp"))
    for i, (shape, axis) in enumerate([((4, 16, 1), -1), ((3, 5, 7, 9), 2), ((2, 8, 28, 28), 3),
                                       ((2, 64, 49), -1), ((6, 1000), 0), ((2, 3, 784), 2)]):
        rng = _rng(400 + i)
        x = _normal(rng, shape)
        oshape = list(shape)
        oshape[axis] = 1
        for op in ("nnc_reducemean", "nnc_reducesum"):
            out.append(case(f"{op}_{i}", op, {"x": x, "out": np.zeros(oshape, F32)},
                            [("t", "x"), ("t", "out"), ("i", axis), ("i", 1)], ["out"], "fp"))
    return out


# --------------------------------------------------------------------------
# pooling
# --------------------------------------------------------------------------
def pool_cases():
    out = []
    # reference tests/test_x86_runtime.py:599-635
    x = np.array([[[[1.0, -2.0, 3.0, 0.5], [2.5, 0.0, -1.0, 4.0], [-3.0, 2.0, 1.0, -0.5],
                    [1.5, -1.5, 2.5, 3.0]],
                   [[-1.0, 0.5, 2.0, -2.5], [3.0, -1.5, 0.25, 1.5], [1.25, 2.5, -3.0, 0.5],
                    [-2.0, 1.0, 1.5, -1.0]]]], F32)
    out.append(case("nnc_maxpool2d_kat", "nnc_maxpool2d",
                    {"x": x, "out": np.zeros((1, 2, 2, 2), F32)},
                    [("t", "x"), ("t", "out"), ("i", 3), ("i", 3), ("i", 2), ("i", 2), ("i", 1), ("i", 1)],
                    ["out"]))
    # empty windows -> -3.402823e38f (reference tests/test_x86_runtime.py:179-193)
    e = np.arange(4, dtype=F32).reshape(1, 1, 2, 2)
    out.append(case("nnc_maxpool2d_empty", "nnc_maxpool2d",
                    {"x": e, "out": np.zeros((1, 1, 10, 10), F32)},
                    [("t", "x"), ("t", "out"), ("i", 1), ("i", 1), ("i", 1), ("i", 1), ("i", 4), ("i", 4)],
                    ["out"]))
    specs = [((2, 3, 11, 12), 3, 3, 2, 2, 1, 1), ((1, 2, 8, 8), 2, 2, 2, 2, 0, 0),
             ((2, 4, 9, 7), 3, 2, 1, 2, 1, 0), ((1, 8, 56, 56), 3, 3, 2, 2, 1, 1)]
    for i, (shape, kh, kw, sh, sw, ph, pw) in enumerate(specs):
        rng = _rng(500 + i)
        x = _normal(rng, shape)
        ho, wo = conv_out_hw(shape[2], shape[3], kh, kw, sh, sw, ph, pw)
        for op in ("nnc_maxpool2d", "nnc_avgpool2d"):
            out.append(case(f"{op}_{i}", op, {"x": x, "out": np.zeros((shape[0], shape[1], ho, wo), F32)},
                            [("t", "x"), ("t", "out"), ("i", kh), ("i", kw), ("i", sh), ("i", sw),
                             ("i", ph), ("i", pw)], ["out"],
                            "exact"))
    # global average pool as emitted (c_emitter.py:373-417): kernel = stride = HxW
    for i, shape in enumerate([(2, 16, 7, 7), (3, 5, 4, 6)]):
        rng = _rng(550 + i)
        x = _normal(rng, shape)
        h, w = shape[2], shape[3]
        out.append(case(f"nnc_avgpool2d_global_{i}", "nnc_avgpool2d",
                        {"x": x, "out": np.zeros((shape[0], shape[1], 1, 1), F32)},
                        [("t", "x"), ("t", "out"), ("i", h), ("i", w), ("i", h), ("i", w), ("i", 0), ("i", 0)],
                        ["out"], "exact"))
    return out


# --------------------------------------------------------------------------
# convolution
# --------------------------------------------------------------------------
_W2 = np.array([[[[0.5, -1.0, 0.25], [1.5, 0.75, -0.5], [-0.25, 0.5, 1.0]],
                 [[-0.75, 0.5, 1.25], [0.0, -1.5, 0.5], [1.0, -0.25, 0.75]]],
                [[[1.0, 0.25, -0.5], [-1.25, 0.5, 0.75], [0.5, -0.75, 1.5]],
                 [[0.25, -1.0, 0.5], [1.5, 0.25, -0.25], [-0.5, 1.0, 0.75]]]], F32)
_B2 = np.array([0.5, -0.25], F32)


def _conv_case(name, op, x, w, b, args_tail, kh, kw, sh, sw, ph, pw, out_shape=None):
    n, _, h, ww = x.shape
    if out_shape is None:
        ho, wo = conv_out_hw(h, ww, kh, kw, sh, sw, ph, pw)
        out_shape = (n, w.shape[0], ho, wo)
    t = {"x": x, "w": w, "out": np.full(out_shape, 3.0, F32)}
    args = [("t", "x"), ("t", "w")]
    if b is None:
        args.append(("null",))
    else:
        t["b"] = b
        args.append(("t", "b"))
    args.append(("t", "out"))
    args += [("i", v) for v in args_tail]
    return case(name, op, t, args, ["out"], "fp")


def conv_cases():
    out = []
    full = lambda kh, kw, sh, sw, ph, pw: [kh, kw, sh, sw, ph, pw]  # noqa: E731
    # literal KATs, reference tests/test_x86_runtime.py:637-1185
    x5 = np.arange(1, 26, dtype=F32).reshape(1, 1, 5, 5)
    w5 = np.array([[[[1.0, 0.0, -1.0], [0.5, 0.25, -0.5], [1.5, -0.25, 0.75]]]], F32)
    out.append(_conv_case("nnc_conv_kat_nopad", "nnc_conv", x5, w5, np.array([0.75], F32),
                          full(3, 3, 1, 1, 0, 0), 3, 3, 1, 1, 0, 0))
    xs = np.array([[[[1.0, -2.0, 3.0, 0.5, -1.5], [2.5, 0.0, -1.0, 4.0, 1.5],
                     [-3.0, 2.0, 1.0, -0.5, 2.5], [1.5, -1.5, 2.5, 3.0, -2.0],
                     [0.25, 1.25, -2.5, 0.75, 1.0]],
                    [[-1.0, 0.5, 2.0, -2.5, 1.0], [3.0, -1.5, 0.25, 1.5, -0.75],
                     [1.25, 2.5, -3.0, 0.5, 2.0], [-2.0, 1.0, 1.5, -1.0, 0.25],
                     [0.5, -0.5, 2.25, 1.75, -1.25]]]], F32)
    out.append(_conv_case("nnc_conv_kat_same", "nnc_conv", xs, _W2, _B2, full(3, 3, 1, 1, 1, 1),
                          3, 3, 1, 1, 1, 1))
    xw = np.arange(1, 1 + 2 * 6 * 10, dtype=F32).reshape(1, 2, 6, 10)
    out.append(_conv_case("nnc_conv_kat_same_wide", "nnc_conv", xw, _W2, _B2, full(3, 3, 1, 1, 1, 1),
                          3, 3, 1, 1, 1, 1))
    x6 = np.array([[[[1.0, -2.0, 3.0, 0.5, -1.5, 2.0], [2.5, 0.0, -1.0, 4.0, 1.5, -0.25],
                     [-3.0, 2.0, 1.0, -0.5, 2.5, 1.25], [1.5, -1.5, 2.5, 3.0, -2.0, 0.75],
                     [0.25, 1.25, -2.5, 0.75, 1.0, -1.0], [2.0, -0.75, 1.5, -2.0, 0.5, 3.0]],
                    [[-1.0, 0.5, 2.0, -2.5, 1.0, 0.25], [3.0, -1.5, 0.25, 1.5, -0.75, 2.25],
                     [1.25, 2.5, -3.0, 0.5, 2.0, -1.5], [-2.0, 1.0, 1.5, -1.0, 0.25, 1.75],
                     [0.5, -0.5, 2.25, 1.75, -1.25, 0.0], [1.5, -2.25, 0.75, 2.5, -0.5, 1.0]]]], F32)
    out.append(_conv_case("nnc_conv_kat_s2", "nnc_conv", x6, _W2, _B2, full(3, 3, 2, 2, 1, 1),
                          3, 3, 2, 2, 1, 1))
    x8 = np.arange(1, 1 + 2 * 8 * 12, dtype=F32).reshape(1, 2, 8, 12)
    out.append(_conv_case("nnc_conv_kat_s2_wide", "nnc_conv", x8, _W2, _B2, full(3, 3, 2, 2, 1, 1),
                          3, 3, 2, 2, 1, 1))
    x1 = np.array([[[[1.0, 2.0], [3.0, 4.0]], [[-1.0, -2.0], [-3.0, -4.0]]]], F32)
    w1 = np.array([[[[2.0]], [[-1.0]]], [[[0.5]], [[3.0]]]], F32)
    b1 = np.array([0.25, -0.5], F32)
    out.append(_conv_case("nnc_conv_kat_1x1", "nnc_conv", x1, w1, b1, full(1, 1, 1, 1, 0, 0),
                          1, 1, 1, 1, 0, 0))
    out.append(_conv_case("nnc_conv1x1_kat", "nnc_conv1x1", x1, w1, b1, [1, 1, 0, 0], 1, 1, 1, 1, 0, 0))
    out.append(_conv_case("nnc_conv_relu1x1_kat", "nnc_conv_relu1x1", x1, w1, b1, [1, 1, 0, 0],
                          1, 1, 1, 1, 0, 0))
    x56 = np.arange(1, 1 + 2 * 5 * 6, dtype=F32).reshape(1, 2, 5, 6)
    out.append(_conv_case("nnc_conv3x3_s1_kat", "nnc_conv3x3_s1", x56, _W2, _B2, [], 3, 3, 1, 1, 1, 1))
    out.append(_conv_case("nnc_conv_relu3x3_s1_kat", "nnc_conv_relu3x3_s1", x56, _W2, _B2, [],
                          3, 3, 1, 1, 1, 1))
    x9 = np.arange(1, 1 + 3 * 9 * 9, dtype=F32).reshape(1, 3, 9, 9)
    w7 = (np.arange(1, 1 + 2 * 3 * 7 * 7, dtype=F32).reshape(2, 3, 7, 7) / F32(50.0)).astype(F32)
    b7 = np.array([0.5, -1.25], F32)
    out.append(_conv_case("nnc_conv7x7_s2_kat", "nnc_conv7x7_s2", x9, w7, b7, [], 7, 7, 2, 2, 3, 3))
    out.append(_conv_case("nnc_conv_relu7x7_s2_kat", "nnc_conv_relu7x7_s2", x9, w7, b7, [],
                          7, 7, 2, 2, 3, 3))

    # seeded cases over every path and the ResNet-18 / LeNet-5 layer kinds
    specs = [
        # name, op, (N,Ci,H,W), Co, kh, kw, sh, sw, ph, pw, bias
        ("r3s1", "nnc_conv", (2, 5, 9, 10), 6, 3, 3, 1, 1, 1, 1, True),
        ("r3s2", "nnc_conv", (2, 4, 11, 9), 7, 3, 3, 2, 2, 1, 1, True),
        ("r1s2", "nnc_conv", (2, 8, 10, 10), 12, 1, 1, 2, 2, 0, 0, True),
        ("stem", "nnc_conv", (1, 3, 22, 20), 8, 7, 7, 2, 2, 3, 3, True),
        ("lenet1", "nnc_conv", (1, 1, 28, 28), 6, 5, 5, 1, 1, 2, 2, True),
        ("lenet2", "nnc_conv", (1, 6, 14, 14), 16, 5, 5, 1, 1, 0, 0, True),
        ("nobias", "nnc_conv", (1, 3, 7, 8), 5, 3, 3, 1, 1, 1, 1, False),
        ("rect", "nnc_conv", (1, 3, 9, 13), 4, 3, 5, 2, 1, 1, 2, True),
        ("relu", "nnc_conv_relu", (2, 6, 8, 8), 9, 3, 3, 1, 1, 1, 1, True),
        ("sigmoid", "nnc_conv_sigmoid", (1, 4, 6, 7), 5, 3, 3, 1, 1, 1, 1, True),
        ("deep", "nnc_conv", (1, 64, 7, 7), 40, 3, 3, 1, 1, 1, 1, True),
        ("wideco", "nnc_conv_relu", (1, 16, 14, 14), 130, 3, 3, 1, 1, 1, 1, True),
    ]
    for i, (tag, op, (n, ci, h, w), co, kh, kw, sh, sw, ph, pw, has_b) in enumerate(specs):
        rng = _rng(600 + i)
        x = _normal(rng, (n, ci, h, w))
        wt = _normal(rng, (co, ci, kh, kw), np.sqrt(2.0 / (ci * kh * kw)))
        b = _normal(rng, (co,), 0.1) if has_b else None
        out.append(_conv_case(f"{op}_{tag}", op, x, wt, b, full(kh, kw, sh, sw, ph, pw),
                              kh, kw, sh, sw, ph, pw))
    # specialised entry points on seeded data
    rng = _rng(650)
    x = _normal(rng, (2, 6, 9, 9))
    w = _normal(rng, (7, 6, 1, 1))
    b = _normal(rng, (7,), 0.1)
    out.append(_conv_case("nnc_conv1x1_pad1", "nnc_conv1x1", x, w, b, [1, 1, 1, 1], 1, 1, 1, 1, 1, 1))
    out.append(_conv_case("nnc_conv1x1_s2", "nnc_conv_relu1x1", x, w, b, [2, 2, 0, 0], 1, 1, 2, 2, 0, 0))
    w3 = _normal(rng, (5, 6, 3, 3), 0.2)
    out.append(_conv_case("nnc_conv3x3_s1_rand", "nnc_conv3x3_s1", x, w3, b[:5].copy(), [],
                          3, 3, 1, 1, 1, 1))
    # shape mismatch: 3x3_s1 must leave the output untouched (ops.c:1089-1093)
    out.append(_conv_case("nnc_conv3x3_s1_mismatch", "nnc_conv3x3_s1", x, w3, None, [],
                          3, 3, 1, 1, 1, 1, out_shape=(2, 5, 7, 7)))
    x7 = _normal(rng, (1, 3, 16, 18))
    w7r = _normal(rng, (6, 3, 7, 7), 0.1)
    out.append(_conv_case("nnc_conv7x7_s2_rand", "nnc_conv_relu7x7_s2", x7, w7r, None, [],
                          7, 7, 2, 2, 3, 3))
    return out


# --------------------------------------------------------------------------
# matrix products
# --------------------------------------------------------------------------
def matmul_cases():
    out = []
    # reference tests/test_x86_runtime.py:1187-1292
    a = np.array([[1.0, 2.0, 3.0], [4.0, 5.0, 6.0]], F32)
    b = np.array([[7.0, 8.0], [9.0, 10.0], [11.0, 12.0]], F32)
    out.append(case("nnc_matmul_kat_2d", "nnc_matmul", {"a": a, "b": b, "out": np.zeros((2, 2), F32)},
                    [("t", "a"), ("t", "b"), ("t", "out")], ["out"], "fp"))
    v = np.array([1.0, 2.0, 3.0], F32)
    m = np.array([[4.0, 5.0], [6.0, 7.0], [8.0, 9.0]], F32)
    out.append(case("nnc_matmul_kat_vm", "nnc_matmul", {"a": v, "b": m, "out": np.zeros((2,), F32)},
                    [("t", "a"), ("t", "b"), ("t", "out")], ["out"], "fp"))
    out.append(case("nnc_matmul_kat_mv", "nnc_matmul",
                    {"a": a, "b": np.array([7.0, 8.0, 9.0], F32), "out": np.zeros((2,), F32)},
                    [("t", "a"), ("t", "b"), ("t", "out")], ["out"], "fp"))
    ga = np.array([[1.0, 2.0, 3.0], [0.5, -1.0, 4.0]], F32)
    gb = np.array([[1.0, 0.0, -1.0], [2.0, 1.0, 0.5], [0.5, -0.25, 3.0], [4.0, 2.0, -2.0]], F32)
    gc = np.array([0.25, -0.5, 1.25, 0.75], F32)
    out.append(case("nnc_gemm_kat_tb", "nnc_gemm", {"a": ga, "b": gb, "c": gc, "out": np.zeros((2, 4), F32)},
                    [("t", "a"), ("t", "b"), ("t", "c"), ("t", "out"), ("f", 1.0), ("f", 1.0),
                     ("i", 0), ("i", 1)], ["out"], "fp"))
    out.append(case("nnc_gemm_nt_kat", "nnc_gemm_nt", {"a": ga, "b": gb, "c": gc, "out": np.zeros((2, 4), F32)},
                    [("t", "a"), ("t", "b"), ("t", "c"), ("t", "out"), ("f", 1.0), ("f", 1.0)],
                    ["out"], "fp"))
    # seeded matmul shapes
    specs = [
        ("2d", (37, 53), (53, 29), (37, 29)),
        ("2d_big", (64, 256), (256, 96), (64, 96)),
        ("vm", (300,), (300, 70), (70,)),
        ("mv", (45, 130), (130,), (45,)),
        ("gemv", (1, 256), (256, 192), (1, 192)),
        ("b1", (1, 16, 32), (1, 32, 24), (1, 16, 24)),
        ("bcastB", (3, 8, 12), (12, 10), (3, 8, 10)),
        ("batched", (4, 9, 16), (4, 16, 11), (4, 9, 11)),
        ("batched4d", (2, 3, 8, 16), (2, 3, 16, 8), (2, 3, 8, 8)),
    ]
    for i, (tag, sa, sb, so) in enumerate(specs):
        rng = _rng(700 + i)
        a = rng.uniform(-1, 1, sa).astype(F32)
        b = rng.uniform(-1, 1, sb).astype(F32)
        extra = {}
        if len(sa) >= 3 and int(np.prod(so[:-2])) > 1:
            extra["hip"] = "batched"
        out.append(case(f"nnc_matmul_{tag}", "nnc_matmul", {"a": a, "b": b, "out": np.zeros(so, F32)},
                        [("t", "a"), ("t", "b"), ("t", "out")], ["out"], "fp", **extra))
    rng = _rng(750)
    a = rng.uniform(-1, 1, (20, 40)).astype(F32)
    b = rng.uniform(-1, 1, (40, 30)).astype(F32)
    out.append(case("nnc_matmul_relu_2d", "nnc_matmul_relu", {"a": a, "b": b, "out": np.zeros((20, 30), F32)},
                    [("t", "a"), ("t", "b"), ("null",), ("t", "out")], ["out"], "fp"))
    # gemm variants: trans flags, bias shapes, alpha/beta
    gspecs = [
        ("nn_bN", 33, 47, 29, 0, 0, "N", 1.0, 1.0),
        ("nt_bN", 32, 64, 100, 0, 1, "N", 1.0, 1.0),
        ("tn_bMN", 17, 23, 31, 1, 0, "MN", 0.5, 2.0),
        ("tt_none", 12, 19, 7, 1, 1, None, 1.5, 0.0),
        ("fc", 2, 512, 200, 0, 1, "N", 1.0, 1.0),
        ("sq", 128, 128, 128, 0, 0, "N", 1.0, 1.0),
    ]
    for i, (tag, M, K, N, ta, tb, cb, alpha, beta) in enumerate(gspecs):
        rng = _rng(760 + i)
        a = rng.uniform(-1, 1, (K, M) if ta else (M, K)).astype(F32)
        b = rng.uniform(-1, 1, (N, K) if tb else (K, N)).astype(F32)
        t = {"a": a, "b": b, "out": np.zeros((M, N), F32)}
        args = [("t", "a"), ("t", "b")]
        if cb is None:
            args.append(("null",))
        else:
            t["c"] = rng.uniform(-1, 1, (N,) if cb == "N" else (M, N)).astype(F32)
            args.append(("t", "c"))
        args += [("t", "out"), ("f", alpha), ("f", beta), ("i", ta), ("i", tb)]
        out.append(case(f"nnc_gemm_{tag}", "nnc_gemm", t, args, ["out"], "fp"))
    for i, (M, K, N) in enumerate([(3, 70, 45), (16, 256, 200)]):
        rng = _rng(780 + i)
        t = {"a": rng.uniform(-1, 1, (M, K)).astype(F32), "b": rng.uniform(-1, 1, (N, K)).astype(F32),
             "c": rng.uniform(-1, 1, (N,)).astype(F32), "out": np.zeros((M, N), F32)}
        out.append(case(f"nnc_gemm_nt_{i}", "nnc_gemm_nt", t,
                        [("t", "a"), ("t", "b"), ("t", "c"), ("t", "out"), ("f", 1.0), ("f", 1.0)],
                        ["out"], "fp"))
    return out


# --------------------------------------------------------------------------
# data movement
# --------------------------------------------------------------------------
def movement_cases():
    out = []
    # reference tests/test_x86_runtime.py:1294-1421
    a = np.array([[1.0, 2.0, 3.0], [4.0, 5.0, 6.0]], F32)
    out.append(case("nnc_transpose_kat", "nnc_transpose", {"x": a, "out": np.zeros((3, 2), F32)},
                    [("t", "x"), ("t", "out"), ("i64", [1, 0]), ("i", 2)], ["out"]))
    a3 = np.arange(24).reshape(2, 3, 4).astype(F32)
    out.append(case("nnc_transpose_kat_3d", "nnc_transpose", {"x": a3, "out": np.zeros((4, 2, 3), F32)},
                    [("t", "x"), ("t", "out"), ("i64", [2, 0, 1]), ("i", 3)], ["out"]))
    r = np.arange(12).reshape(3, 4).astype(F32)
    out.append(case("nnc_reshape_kat", "nnc_reshape", {"x": r, "out": np.zeros((2, 6), F32)},
                    [("t", "x"), ("t", "out"), ("i64", [2, 6]), ("i", 2)], ["out"]))
    c1 = np.array([[1.0, 2.0], [3.0, 4.0]], F32)
    c2 = np.array([[5.0, 6.0], [7.0, 8.0]], F32)
    out.append(case("nnc_concat_kat_a0", "nnc_concat", {"a": c1, "b": c2, "out": np.zeros((4, 2), F32)},
                    [("tl", ["a", "b"]), ("t", "out"), ("i", 2), ("i", 0)], ["out"]))
    out.append(case("nnc_concat_kat_a1", "nnc_concat", {"a": c1, "b": c2, "out": np.zeros((2, 4), F32)},
                    [("tl", ["a", "b"]), ("t", "out"), ("i", 2), ("i", 1)], ["out"]))
    s = np.array([[1.0, 2.0, 3.0, 4.0], [5.0, 6.0, 7.0, 8.0]], F32)
    out.append(case("nnc_split_kat", "nnc_split",
                    {"x": s, "o1": np.zeros((2, 2), F32), "o2": np.zeros((2, 2), F32)},
                    [("t", "x"), ("tl", ["o1", "o2"]), ("i", 2), ("i", 1)], ["o1", "o2"]))
    tl = np.array([[1.0, 2.0], [3.0, 4.0]], F32)
    out.append(case("nnc_tile_kat_2d", "nnc_tile", {"x": tl, "out": np.zeros((4, 6), F32)},
                    [("t", "x"), ("t", "out"), ("i64", [2, 3]), ("i", 2)], ["out"]))
    t1 = np.array([1.0, 2.0, 3.0], F32)
    out.append(case("nnc_tile_kat_1d", "nnc_tile", {"x": t1, "out": np.zeros((12,), F32)},
                    [("t", "x"), ("t", "out"), ("i64", [4]), ("i", 1)], ["out"]))
    # seeded
    rng = _rng(800)
    x4 = _normal(rng, (2, 5, 6, 7))
    for i, perm in enumerate([(0, 2, 1, 3), (0, 1, 3, 2), (3, 2, 1, 0), (1, 0, 2, 3), (0, 2, 3, 1)]):
        oshape = tuple(x4.shape[p] for p in perm)
        out.append(case(f"nnc_transpose_4d_{i}", "nnc_transpose", {"x": x4, "out": np.zeros(oshape, F32)},
                        [("t", "x"), ("t", "out"), ("i64", list(perm)), ("i", 4)], ["out"]))
    out.append(case("nnc_transpose_null", "nnc_transpose",
                    {"x": x4, "out": np.zeros(x4.shape[::-1], F32)},
                    [("t", "x"), ("t", "out"), ("i64null",), ("i", 4)], ["out"]))
    big = _normal(rng, (2, 4, 32, 64))
    out.append(case("nnc_transpose_heads", "nnc_transpose",
                    {"x": big, "out": np.zeros((2, 32, 4, 64), F32)},
                    [("t", "x"), ("t", "out"), ("i64", [0, 2, 1, 3]), ("i", 4)], ["out"]))
    m2 = _normal(rng, (130, 67))
    out.append(case("nnc_transpose_2d_odd", "nnc_transpose", {"x": m2, "out": np.zeros((67, 130), F32)},
                    [("t", "x"), ("t", "out"), ("i64", [1, 0]), ("i", 2)], ["out"]))
    f = _normal(rng, (3, 4, 1, 1))
    out.append(case("nnc_flatten_0", "nnc_flatten", {"x": f, "out": np.zeros((3, 4), F32)},
                    [("t", "x"), ("t", "out"), ("i", 1)], ["out"]))
    out.append(case("nnc_squeeze_0", "nnc_squeeze", {"x": f, "out": np.zeros((3, 4, 1), F32)},
                    [("t", "x"), ("t", "out"), ("i", 3)], ["out"]))
    out.append(case("nnc_unsqueeze_0", "nnc_unsqueeze", {"x": m2, "out": np.zeros((1, 130, 67), F32)},
                    [("t", "x"), ("t", "out"), ("i", 0)], ["out"]))
    out.append(case("nnc_identity_0", "nnc_identity", {"x": m2, "out": np.zeros_like(m2)},
                    [("t", "x"), ("t", "out")], ["out"]))
    out.append(case("nnc_identity_short", "nnc_identity",
                    {"x": m2[:10].copy(), "out": np.full((20, 67), 5.0, F32)},
                    [("t", "x"), ("t", "out")], ["out"]))
    ca, cb, cc = _normal(rng, (2, 3, 4, 5)), _normal(rng, (2, 1, 4, 5)), _normal(rng, (2, 6, 4, 5))
    out.append(case("nnc_concat_a1", "nnc_concat",
                    {"a": ca, "b": cb, "c": cc, "out": np.zeros((2, 10, 4, 5), F32)},
                    [("tl", ["a", "b", "c"]), ("t", "out"), ("i", 3), ("i", 1)], ["out"]))
    out.append(case("nnc_concat_last", "nnc_concat",
                    {"a": ca, "b": ca.copy(), "out": np.zeros((2, 3, 4, 10), F32)},
                    [("tl", ["a", "b"]), ("t", "out"), ("i", 2), ("i", -1)], ["out"]))
    ia = np.arange(6, dtype=np.int64).reshape(2, 3)
    ib = np.arange(100, 104, dtype=np.int64).reshape(2, 2)
    out.append(case("nnc_concat_i64", "nnc_concat",
                    {"a": ia, "b": ib, "out": np.zeros((2, 5), np.int64)},
                    [("tl", ["a", "b"]), ("t", "out"), ("i", 2), ("i", 1)], ["out"]))
    sx = _normal(rng, (2, 12, 3, 5))
    out.append(case("nnc_split_a1_3", "nnc_split",
                    {"x": sx, "o1": np.zeros((2, 4, 3, 5), F32), "o2": np.zeros((2, 4, 3, 5), F32),
                     "o3": np.zeros((2, 4, 3, 5), F32)},
                    [("t", "x"), ("tl", ["o1", "o2", "o3"]), ("i", 3), ("i", 1)], ["o1", "o2", "o3"]))
    si = np.arange(24, dtype=np.int64).reshape(4, 6)
    out.append(case("nnc_split_i64", "nnc_split",
                    {"x": si, "o1": np.zeros((2, 6), np.int64), "o2": np.zeros((2, 6), np.int64)},
                    [("t", "x"), ("tl", ["o1", "o2"]), ("i", 2), ("i", 0)], ["o1", "o2"]))
    ex = _normal(rng, (4,))
    out.append(case("nnc_expand_0", "nnc_expand", {"x": ex, "out": np.zeros((3, 4), F32)},
                    [("t", "x"), ("t", "out"), ("i64", [3, 4]), ("i", 2)], ["out"]))
    out.append(case("nnc_tile_3d", "nnc_tile", {"x": ca[0], "out": np.zeros((6, 4, 10), F32)},
                    [("t", "x"), ("t", "out"), ("i64", [2, 1, 2]), ("i", 3)], ["out"]))
    return out


def misc_cases():
    out = []
    rng = _rng(900)
    x = (_normal(rng, (3, 11)) * 5).astype(F32)
    x.ravel()[:4] = [0.0, -0.0, 2.5, -2.5]
    for to, dt in [(2, np.int32), (6, np.int64), (5, np.uint8), (0, F32)]:
        out.append(case(f"nnc_cast_f32_to_{to}", "nnc_cast", {"x": x, "out": np.zeros(x.shape, dt)},
                        [("t", "x"), ("t", "out"), ("i", to)], ["out"]))
    bx = rng.random((2, 9)) > 0.5  # numpy bool -> NNC_DTYPE_BOOL
    bt = {"x": bx}
    for to, dt in [(0, F32), (2, np.int32), (6, np.int64), (5, np.uint8)]:
        t = dict(bt)
        t["out"] = np.zeros(bx.shape, dt)
        out.append(case(f"nnc_cast_bool_to_{to}", "nnc_cast", t,
                        [("t", "x"), ("t", "out"), ("i", to)], ["out"]))
    sx = np.zeros((2, 3, 5), F32)
    out.append(case("nnc_shape_rt", "nnc_shape", {"x": sx, "out": np.zeros((3,), np.int64)},
                    [("t", "x"), ("t", "out"), ("i64null",), ("i", 3)], ["out"]))
    out.append(case("nnc_shape_ct", "nnc_shape", {"x": sx, "out": np.zeros((3,), np.int64)},
                    [("t", "x"), ("t", "out"), ("i64", [7, 8, 9]), ("i", 3)], ["out"]))
    out.append(case("nnc_constantofshape_0", "nnc_constantofshape", {"out": np.zeros((4, 7), F32)},
                    [("t", "out"), ("f", 2.5), ("i", 2)], ["out"]))
    # gather: scalar index rank 2, 1-D indices rank 2 axis 0 / 1, rank 3 axes, int64 data
    d2 = _normal(rng, (6, 5))
    d3 = _normal(rng, (4, 3, 5))
    i1 = np.array([-1], np.int64)
    iv = np.array([4, 0, -2, 9], np.int64)
    gspecs = [
        ("s2a0", d2, i1, (1, 5), 0, 0), ("s2a1", d2, np.array([2], np.int64), (6, 1), 1, 0),
        ("v2a0", d2, iv, (4, 5), 0, 0), ("v2a1", d2, np.array([1, 3], np.int64), (6, 2), 1, 0),
        ("s3a0", d3, np.array([2], np.int64), (3, 5), 0, 0), ("s3a1", d3, np.array([1], np.int64), (4, 5), 1, 0),
        ("s3a2", d3, np.array([3], np.int64), (4, 3), 2, 0), ("s1", np.arange(7, dtype=F32), np.array([5], np.int64), (3,), 0, 0),
    ]
    for tag, d, ix, oshape, axis, dd in gspecs:
        out.append(case(f"nnc_gather_{tag}", "nnc_gather",
                        {"d": d, "ix": ix, "out": np.zeros(oshape, F32)},
                        [("t", "d"), ("t", "ix"), ("t", "out"), ("i", axis), ("i", dd)], ["out"]))
    di = np.array([10, 20, 30, 40], np.int64)
    out.append(case("nnc_gather_i64_v", "nnc_gather",
                    {"d": di, "ix": np.array([3, -1, 0], np.int64), "out": np.zeros((3,), np.int64)},
                    [("t", "d"), ("t", "ix"), ("t", "out"), ("i", 0), ("i", 1)], ["out"]))
    # LSTM: forward and bidirectional, with and without bias
    for tag, T, B, I, H, dirn, has_b in [("fwd", 3, 2, 4, 5, 0, True), ("bidir", 4, 1, 3, 6, 2, True),
                                         ("rev_nob", 2, 2, 5, 4, 1, False)]:
        rng = _rng(950 + T * 10 + H)
        nd = 2 if dirn == 2 else 1
        t = {"X": _normal(rng, (T, B, I), 0.5), "W": _normal(rng, (nd, 4 * H, I), 0.3),
             "R": _normal(rng, (nd, 4 * H, H), 0.3),
             "Y": np.zeros((T, nd, B, H), F32), "Yh": np.zeros((nd, B, H), F32),
             "Yc": np.zeros((nd, B, H), F32)}
        args = [("t", "X"), ("t", "W"), ("t", "R")]
        if has_b:
            t["B"] = _normal(rng, (nd, 8 * H), 0.1)
            args.append(("t", "B"))
        else:
            args.append(("null",))
        args += [("t", "Y"), ("t", "Yh"), ("t", "Yc"), ("i", dirn), ("i", H)]
        out.append(case(f"nnc_lstm_{tag}", "nnc_lstm", t, args, ["Y", "Yh", "Yc"], "fp"))
    bn = _normal(rng, (2, 3, 4, 4))
    out.append(case("nnc_batchnorm_noop", "nnc_batchnorm",
                    {"x": bn, "s": np.ones(3, F32), "b": np.zeros(3, F32), "m": np.zeros(3, F32),
                     "v": np.ones(3, F32), "out": np.full(bn.shape, 9.0, F32)},
                    [("t", "x"), ("t", "s"), ("t", "b"), ("t", "m"), ("t", "v"), ("t", "out"),
                     ("f", 1e-5), ("i", 0)], ["out"]))
    return out


def all_cases():
    cs = (binary_cases() + unary_cases() + logic_cases() + softmax_cases() + layernorm_cases()
          + reduce_cases() + pool_cases() + conv_cases() + matmul_cases() + movement_cases()
          + misc_cases())
    names = [c["name"] for c in cs]
    assert len(names) == len(set(names)), "duplicate case names"
    return cs
