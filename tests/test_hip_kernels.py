"""Targeted GPU checks of the MFMA kernels at shapes the golden vectors are
too small to reach: every conv tile configuration with stream-K splitting
(tiles fewer than resident workgroups, K tails, 3-channel stem), the fused
conv+add+relu of the mi355x target (also in place over its residual), the
packed-weight direct-to-LDS convolution, and GEMM / MatMul layouts. Expected values come from the oracle on the host, the
same seeded inputs; bar |got - ref| <= 1e-4 or <= 1e-3 * |ref|."""

from __future__ import annotations

import ctypes

import numpy as np
import pytest

import caserun

pytestmark = pytest.mark.gpu

ATOL, RTOL = 1e-4, 1e-3


def _check(got, exp, what):
    bad = caserun.fp_violations(got, exp, ATOL, RTOL)
    assert bad.size == 0, (f"{what}: {bad.size}/{got.size} outside atol {ATOL} / rtol {RTOL}; first "
                           f"{bad[:5]}: got {got.ravel()[bad[:5]]} want {exp.ravel()[bad[:5]]}")


def _conv_case(rng, n, ci, h, co, k, s, p, op="nnc_conv", with_bias=True):
    ho = (h + 2 * p - k) // s + 1
    x = rng.standard_normal((n, ci, h, h)).astype(np.float32)
    w = (rng.standard_normal((co, ci, k, k)) / np.sqrt(ci * k * k)).astype(np.float32)
    b = (rng.standard_normal(co) * 0.1).astype(np.float32)
    out = np.zeros((n, co, ho, ho), np.float32)
    tensors = {"x": x, "w": w, "out": out}
    if with_bias:
        tensors["b"] = b
    args = [("t", "x"), ("t", "w"), ("t", "b") if with_bias else ("null",), ("t", "out"),
            ("i", k), ("i", k), ("i", s), ("i", s), ("i", p), ("i", p)]
    return {"name": f"{op}_{n}x{ci}x{h}_{co}_k{k}s{s}p{p}", "op": op, "tensors": tensors, "args": args,
            "outputs": ["out"], "bar": "fp"}


# (N, Ci, H, Co, k, s, p): ResNet-18 layer shapes at small batch plus edge cases
CONV_SHAPES = [
    (2, 3, 64, 64, 7, 2, 3),      # stem-like: K = 147 (scalar A loads, K tail)
    (2, 64, 28, 64, 3, 1, 1),     # 64-channel 3x3
    (4, 64, 56, 64, 3, 1, 1),     # 64x128 tiles, stream-K
    (8, 128, 28, 128, 3, 1, 1),   # 128x128 tiles, stream-K over 49 tiles x 36 slices
    (2, 256, 14, 512, 3, 2, 1),   # stride 2, many M tiles
    (4, 512, 7, 512, 3, 1, 1),    # K = 4608, few tiles: many partials per tile
    (4, 256, 14, 512, 1, 2, 0),   # 1x1 stride 2
    (3, 5, 11, 7, 3, 1, 1),       # odd sizes everywhere
    (1, 33, 9, 130, 5, 2, 2),     # generic kernel size, K tail, Co tail
    # register-staged 128x128 tiles (Ci % 32 != 0, K = 540): stream-K
    # partials in register order, a Co tail and images straddling tiles
    (2, 60, 24, 136, 3, 1, 1),
]


@pytest.mark.parametrize("shape", CONV_SHAPES, ids=[str(s) for s in CONV_SHAPES])
def test_conv_streamk_shapes(shape, hip, dmem, abi, oracle_lib):
    case = _conv_case(np.random.default_rng(7), *shape, op="nnc_conv_relu")
    print(f"case {case['name']}", flush=True)
    exp = caserun.run_case(oracle_lib, case, abi)["out"]
    got = caserun.run_case(hip, case, abi, dmem)["out"]
    _check(got, exp, case["name"])


FUSED_SHAPES = [
    (2, 64, 28, 64, 3, 1, 1),
    (8, 128, 28, 128, 3, 1, 1),
    (4, 512, 7, 512, 3, 1, 1),
    (4, 128, 28, 256, 1, 2, 0),
]


@pytest.mark.parametrize("shape", FUSED_SHAPES, ids=[str(s) for s in FUSED_SHAPES])
@pytest.mark.parametrize("bias", [True, False])
def test_conv_add_relu_matches_composition(shape, bias, hip, dmem, abi, oracle_lib):
    rng = np.random.default_rng(11)
    case = _conv_case(rng, *shape, op="nnc_hip_conv_add_relu", with_bias=bias)
    case["tensors"]["res"] = rng.standard_normal(case["tensors"]["out"].shape).astype(np.float32)
    case["args"].insert(3, ("t", "res"))
    print(f"case {case['name']} bias={bias}", flush=True)
    exp = caserun.run_case(oracle_lib, case, abi)["out"]
    got = caserun.run_case(hip, case, abi, dmem)["out"]
    _check(got, exp, case["name"])
    # the same as nnc_conv then nnc_add_relu on the GPU, to the bit
    conv = dict(case, op="nnc_conv", args=[a for i, a in enumerate(case["args"]) if i != 3])
    mid = caserun.run_case(hip, conv, abi, dmem)["out"]
    add = {"name": "add", "op": "nnc_add_relu", "tensors": {"a": mid, "b": case["tensors"]["res"],
                                                             "out": np.zeros_like(mid)},
           "args": [("t", "a"), ("t", "b"), ("t", "out")], "outputs": ["out"], "bar": "exact"}
    two = caserun.run_case(hip, add, abi, dmem)["out"]
    assert caserun.same_bits(got, two)


def test_conv_add_relu_in_place_over_residual(hip, abi, oracle_lib):
    from nnc_py_amd import runtime
    rng = np.random.default_rng(5)
    n, ci, h, co = 4, 128, 28, 128
    x = rng.standard_normal((n, ci, h, h)).astype(np.float32)
    w = (rng.standard_normal((co, ci, 3, 3)) / np.sqrt(ci * 9)).astype(np.float32)
    b = (rng.standard_normal(co) * 0.1).astype(np.float32)
    res = rng.standard_normal((n, co, h, h)).astype(np.float32)
    case = {"name": "ref", "op": "nnc_hip_conv_add_relu",
            "tensors": {"x": x, "w": w, "b": b, "res": res, "out": np.zeros_like(res)},
            "args": [("t", "x"), ("t", "w"), ("t", "b"), ("t", "res"), ("t", "out")] +
                    [("i", v) for v in (3, 3, 1, 1, 1, 1)], "outputs": ["out"], "bar": "fp"}
    exp = caserun.run_case(oracle_lib, case, abi)["out"]
    bx, bw, bb = (runtime.DeviceBuffer.from_array(a) for a in (x, w, b))
    bres = runtime.DeviceBuffer.from_array(res)
    tx, tw, tb, tr = bx.tensor(), bw.tensor(), bb.tensor(), bres.tensor()
    hip.nnc_hip_conv_add_relu(ctypes.byref(tx[0]), ctypes.byref(tw[0]), ctypes.byref(tb[0]),
                              ctypes.byref(tr[0]), ctypes.byref(tr[0]), 3, 3, 1, 1, 1, 1)
    runtime.sync()
    assert runtime.last_error()[0] == 0
    _check(bres.to_array(), exp, "in place")


def test_conv_add_relu_rejects_bad_residual(hip, dmem, abi):
    from nnc_py_amd import runtime
    rng = np.random.default_rng(1)
    case = _conv_case(rng, 1, 8, 8, 8, 3, 1, 1, op="nnc_hip_conv_add_relu")
    case["tensors"]["res"] = np.zeros((1, 8, 4, 4), np.float32)  # smaller than the output
    case["args"].insert(3, ("t", "res"))
    runtime.clear_error()
    out = caserun.run_case(hip, case, abi, dmem)["out"]
    assert runtime.last_error()[0] != 0
    assert not out.any()


def _packed_case(rng, n, ci, h, co, k, s, p, act=1, bias=True, res=True, w_ref=None):
    """nnc_hip_conv_packed case: weights drawn in the reference layout and
    passed tap-major [Co][kh][kw][Ci]."""
    ho = (h + 2 * p - k) // s + 1
    x = rng.standard_normal((n, ci, h, h)).astype(np.float32)
    w = (rng.standard_normal((co, ci, k, k)) / np.sqrt(ci * k * k)).astype(np.float32) if w_ref is None else w_ref
    tensors = {"x": x, "w": np.ascontiguousarray(w.transpose(0, 2, 3, 1)),
               "out": np.zeros((n, co, ho, ho), np.float32)}
    if bias:
        tensors["b"] = (rng.standard_normal(co) * 0.1).astype(np.float32)
    if res:
        tensors["res"] = rng.standard_normal((n, co, ho, ho)).astype(np.float32)
    args = [("t", "x"), ("t", "w"), ("t", "b") if bias else ("null",), ("t", "res") if res else ("null",),
            ("t", "out")] + [("i", v) for v in (k, k, s, s, p, p, act)]
    return {"name": f"packed_{n}x{ci}x{h}_{co}_k{k}s{s}p{p}_a{act}{'b' if bias else ''}{'r' if res else ''}",
            "op": "nnc_hip_conv_packed", "tensors": tensors, "args": args, "outputs": ["out"], "bar": "fp"}


# every tile configuration of the direct-to-LDS kernels, tails in Co and
# pixels, stride 2, no padding, 1x1; batches large enough (over 0.5 GFLOP or
# 256 tiles of 64 x 64) that the short-convolution kernel does not take them
PACKED_SHAPES = [
    (32, 32, 28, 64, 3, 1, 1),    # 64x64 tiles (K = 288)
    (4, 64, 56, 64, 3, 1, 1),     # 64x128 tiles, stream-K
    (8, 128, 28, 128, 3, 1, 1),   # 128x128 tiles, stream-K
    (16, 256, 14, 256, 3, 1, 1),  # 128x128 with a partial last pixel tile
    (8, 256, 14, 512, 3, 2, 1),   # stride 2, many M tiles
    (4, 512, 7, 512, 3, 1, 1),    # K = 4608: many partials per tile
    (170, 32, 13, 96, 3, 2, 1),   # odd image, Co and pixel tails
    (7, 64, 19, 198, 3, 1, 1),    # 128x128 tiles: Co % 4 != 0, 2527 pixels of 361-pixel images
    (210, 32, 9, 40, 3, 1, 1),    # Co < tile
    (200, 64, 10, 64, 3, 1, 0),   # no padding
    (64, 64, 14, 128, 1, 1, 0),   # 1x1
    (32, 128, 28, 256, 1, 2, 0),  # 1x1 stride 2
]

# the short-convolution kernel (conv_ws_k: 32x32 tiles, waves splitting K,
# S workgroups per tile finished in-kernel): ResNet-18's layers at batch 1
# (S = 1, 2, 4, 8; 49-pixel images), batch 2 (images straddling tiles),
# tails in Co and pixels, stride 2, no padding, 1x1, a single tile
WS_SHAPES = [
    (1, 64, 56, 64, 3, 1, 1),     # S = 1, five slices per wave
    (1, 64, 56, 128, 3, 2, 1),    # stride 2, S = 1
    (1, 128, 28, 128, 3, 1, 1),   # S = 2
    (1, 256, 14, 256, 3, 1, 1),   # S = 4
    (1, 512, 7, 512, 3, 1, 1),    # S = 8, K = 4608, 49 pixels (scalar stores)
    (2, 512, 7, 512, 3, 1, 1),    # two images across one 32-pixel tile
    (3, 32, 13, 96, 3, 2, 1),     # odd image, pixel tail
    (3, 64, 19, 198, 3, 1, 1),    # Co % 32 != 0
    (2, 32, 9, 40, 3, 1, 1),      # second channel tile of 8 rows
    (2, 64, 10, 64, 3, 1, 0),     # no padding
    (4, 64, 14, 128, 1, 1, 0),    # 1x1
    (4, 128, 28, 256, 1, 2, 0),   # 1x1 stride 2
    (1, 32, 5, 32, 3, 1, 1),      # one tile, 9 slices
]


@pytest.mark.parametrize("shape", PACKED_SHAPES, ids=[str(s) for s in PACKED_SHAPES])
def test_conv_packed_shapes(shape, hip, dmem, abi, oracle_lib):
    case = _packed_case(np.random.default_rng(13), *shape)
    print(f"case {case['name']}", flush=True)
    exp = caserun.run_case(oracle_lib, case, abi)["out"]
    got = caserun.run_case(hip, case, abi, dmem)["out"]
    _check(got, exp, case["name"])


@pytest.mark.parametrize("shape", WS_SHAPES, ids=[str(s) for s in WS_SHAPES])
def test_conv_ws_shapes(shape, hip, dmem, abi, oracle_lib):
    """conv_ws_k against the oracle, and run again on the same input: bit
    for bit the same (the split tiles' sums are added in range order
    whichever workgroup finishes)."""
    case = _packed_case(np.random.default_rng(37), *shape)
    print(f"case {case['name']}", flush=True)
    exp = caserun.run_case(oracle_lib, case, abi)["out"]
    got = caserun.run_case(hip, case, abi, dmem)["out"]
    _check(got, exp, case["name"])
    again = caserun.run_case(hip, case, abi, dmem)["out"]
    assert caserun.same_bits(again, got)


@pytest.mark.parametrize("act", [0, 1, 2])
@pytest.mark.parametrize("bias,res", [(True, True), (False, True), (True, False), (False, False)])
def test_conv_ws_epilogues(act, bias, res, hip, dmem, abi, oracle_lib):
    """Each activation, with and without bias and residual, on a whole tile
    (S = 1) and a split one (S = 8); then on images whose pixel count is not
    a multiple of 4 (a thread's four pixels reach into the next image: 3 x
    7x7, 5 x 3x3) and on 1-pixel images (8 x 1x1 outputs)."""
    for shape in ((1, 64, 12, 64, 3, 1, 1), (1, 512, 7, 512, 3, 1, 1), (3, 64, 7, 64, 3, 1, 1),
                  (5, 32, 3, 64, 3, 1, 1), (8, 32, 3, 64, 3, 1, 0)):
        case = _packed_case(np.random.default_rng(43), *shape, act=act, bias=bias, res=res)
        print(f"case {case['name']}", flush=True)
        exp = caserun.run_case(oracle_lib, case, abi)["out"]
        got = caserun.run_case(hip, case, abi, dmem)["out"]
        _check(got, exp, case["name"])


@pytest.mark.parametrize("n,h", [(2, 64), (1, 224), (3, 37), (2, 224), (1, 560), (5, 224), (16, 64)])
def test_conv_packed_stem(n, h, hip, dmem, abi, oracle_lib):
    """3-channel 7x7 stride-2 stem on [Co][Kp] rows (K = 147 padded to 160):
    64x64 tiles (2 x 64x64, 1 x 224x224, 3 x 37x37, 2 x 224x224), 64x128
    tiles from 65536 output pixels (1 x 560x560: 280 rows); from 512 output
    rows on (5 x 224x224, 16 x 64x64) the row kernel with its input window
    in LDS."""
    rng = np.random.default_rng(23)
    case = _packed_case(rng, n, 3, h, 64, 7, 2, 3, res=False)
    w = case["tensors"]["w"]  # [Co][7][7][3]
    rows = np.zeros((64, 160), np.float32)
    rows[:, :147] = w.reshape(64, 147)
    case["tensors"]["w"] = rows
    print(f"case {case['name']}", flush=True)
    exp = caserun.run_case(oracle_lib, case, abi)["out"]
    got = caserun.run_case(hip, case, abi, dmem)["out"]
    _check(got, exp, case["name"])


@pytest.mark.parametrize("n,h,co,act,bias", [(1, 224, 40, 2, False), (1, 64, 16, 1, True), (2, 96, 64, 0, True)])
def test_conv_stem_tile_epilogues(n, h, co, act, bias, hip, dmem, abi, oracle_lib):
    """The stem on 64x64 tiles with fewer output channels than a tile's 64
    rows (40, 16: weight rows past Co read as zeros, their stores skipped),
    each activation, with and without bias."""
    rng = np.random.default_rng(31)
    case = _packed_case(rng, n, 3, h, co, 7, 2, 3, act=act, bias=bias, res=False)
    w = case["tensors"]["w"]
    rows = np.zeros((co, 160), np.float32)
    rows[:, :147] = w.reshape(co, 147)
    case["tensors"]["w"] = rows
    print(f"case {case['name']}", flush=True)
    exp = caserun.run_case(oracle_lib, case, abi)["out"]
    got = caserun.run_case(hip, case, abi, dmem)["out"]
    _check(got, exp, case["name"])


@pytest.mark.parametrize("co,act,bias", [(40, 2, False), (64, 0, True), (16, 1, True)])
def test_conv_stem_rows_epilogues(co, act, bias, hip, dmem, abi, oracle_lib):
    """The row kernel (16 x 64x64 images: 512 output rows) with fewer than 64
    output channels (weight rows past Co read as zeros, their stores
    skipped), each activation, with and without bias."""
    rng = np.random.default_rng(29)
    case = _packed_case(rng, 16, 3, 64, co, 7, 2, 3, act=act, bias=bias, res=False)
    w = case["tensors"]["w"]
    rows = np.zeros((co, 160), np.float32)
    rows[:, :147] = w.reshape(co, 147)
    case["tensors"]["w"] = rows
    print(f"case {case['name']}", flush=True)
    exp = caserun.run_case(oracle_lib, case, abi)["out"]
    got = caserun.run_case(hip, case, abi, dmem)["out"]
    _check(got, exp, case["name"])


def _proj_case(rng, n, ci, h, co, cx, xh, ps, act=1, bias=True):
    """nnc_hip_conv_proj case: 3x3 / stride 1 / pad 1 over x [n, ci, h, h]
    plus a 1x1 stride-ps projection of p [n, cx, xh, xh]; weights drawn in
    the reference layout, packed [Co][9*Ci + Cx]."""
    x = rng.standard_normal((n, ci, h, h)).astype(np.float32)
    pin = rng.standard_normal((n, cx, xh, xh)).astype(np.float32)
    w3 = (rng.standard_normal((co, ci, 3, 3)) / np.sqrt(ci * 9)).astype(np.float32)
    w1 = (rng.standard_normal((co, cx, 1, 1)) / np.sqrt(cx)).astype(np.float32)
    rows = np.concatenate([w3.transpose(0, 2, 3, 1).reshape(co, -1), w1.reshape(co, cx)], axis=1)
    tensors = {"x": x, "w": np.ascontiguousarray(rows), "p": pin, "out": np.zeros((n, co, h, h), np.float32)}
    if bias:
        tensors["b"] = (rng.standard_normal(co) * 0.1).astype(np.float32)
    args = [("t", "x"), ("t", "w"), ("t", "b") if bias else ("null",), ("t", "p"), ("t", "out")]
    args += [("i", v) for v in (3, 3, 1, 1, 1, 1, ps, ps, act)]
    return {"name": f"proj_{n}x{ci}x{h}_{co}_p{cx}x{xh}s{ps}_a{act}{'b' if bias else ''}",
            "op": "nnc_hip_conv_proj", "tensors": tensors, "args": args, "outputs": ["out"], "bar": "fp"}


# every tile configuration (64x64, 64x128 with the in-kernel finish, 128x128),
# ResNet-18's three downsample blocks at batch 1 and 32, a stride-1
# projection, odd images and Co / pixel tails
PROJ_SHAPES = [
    (2, 64, 28, 64, 32, 56, 2),
    (4, 64, 56, 64, 64, 112, 2),
    (8, 128, 28, 128, 64, 56, 2),
    (1, 128, 28, 128, 64, 56, 2),
    (1, 512, 7, 512, 256, 14, 2),
    (32, 256, 14, 256, 128, 28, 2),
    (3, 32, 13, 96, 32, 13, 1),
    (2, 64, 9, 40, 96, 17, 2),
]


@pytest.mark.parametrize("shape", PROJ_SHAPES, ids=[str(s) for s in PROJ_SHAPES])
def test_conv_proj_shapes(shape, hip, dmem, abi, oracle_lib):
    case = _proj_case(np.random.default_rng(29), *shape)
    print(f"case {case['name']}", flush=True)
    exp = caserun.run_case(oracle_lib, case, abi)["out"]
    got = caserun.run_case(hip, case, abi, dmem)["out"]
    _check(got, exp, case["name"])


@pytest.mark.parametrize("act", [0, 1, 2])
@pytest.mark.parametrize("bias", [True, False])
def test_conv_proj_epilogues(act, bias, hip, dmem, abi, oracle_lib):
    for shape in ((2, 64, 12, 64, 32, 24, 2), (8, 128, 28, 128, 64, 56, 2)):
        case = _proj_case(np.random.default_rng(31), *shape, act=act, bias=bias)
        print(f"case {case['name']}", flush=True)
        exp = caserun.run_case(oracle_lib, case, abi)["out"]
        got = caserun.run_case(hip, case, abi, dmem)["out"]
        _check(got, exp, case["name"])


@pytest.mark.parametrize("why,cx,xh,cols", [("Cx not a multiple of 32", 48, 24, None),
                                            ("projection input too small", 32, 22, None),
                                            ("weight rows of the wrong length", 32, 24, 9 * 64 + 16)])
def test_conv_proj_rejects(why, cx, xh, cols, hip, dmem, abi):
    """Refused on the host (error code, nothing launched, output untouched)."""
    from nnc_py_amd import runtime
    case = _proj_case(np.random.default_rng(3), 2, 64, 12, 64, cx, xh, 2)
    if cols is not None:
        case["tensors"]["w"] = np.zeros((64, cols), np.float32)
    runtime.clear_error()
    out = caserun.run_case(hip, case, abi, dmem)["out"]
    assert runtime.last_error()[0] != 0, why
    assert not out.any()
    runtime.clear_error()


@pytest.mark.parametrize("act", [0, 1, 2])
@pytest.mark.parametrize("bias,res", [(True, False), (False, True), (False, False)])
def test_conv_packed_epilogues(act, bias, res, hip, dmem, abi, oracle_lib):
    for shape in ((2, 64, 12, 64, 3, 1, 1), (8, 128, 28, 128, 3, 1, 1)):
        case = _packed_case(np.random.default_rng(17), *shape, act=act, bias=bias, res=res)
        print(f"case {case['name']}", flush=True)
        exp = caserun.run_case(oracle_lib, case, abi)["out"]
        got = caserun.run_case(hip, case, abi, dmem)["out"]
        _check(got, exp, case["name"])


def test_conv_packed_matches_reference_layout_entry(hip, dmem, abi, oracle_lib):
    """The packed entry on transposed weights agrees with nnc_conv_relu on
    the original ones (both within the bar of the oracle's fp64 sums)."""
    rng = np.random.default_rng(19)
    packed = _packed_case(rng, 4, 128, 28, 128, 3, 1, 1, bias=True, res=False)
    w = np.ascontiguousarray(packed["tensors"]["w"].transpose(0, 3, 1, 2))
    plain = {"name": "plain", "op": "nnc_conv_relu",
             "tensors": {"x": packed["tensors"]["x"], "w": w, "b": packed["tensors"]["b"],
                         "out": np.zeros_like(packed["tensors"]["out"])},
             "args": [("t", "x"), ("t", "w"), ("t", "b"), ("t", "out")] + [("i", v) for v in (3, 3, 1, 1, 1, 1)],
             "outputs": ["out"], "bar": "fp"}
    got = caserun.run_case(hip, packed, abi, dmem)["out"]
    ref = caserun.run_case(hip, plain, abi, dmem)["out"]
    _check(got, ref, "packed vs reference layout")


@pytest.mark.parametrize("why,shape,wshape", [
    ("Ci % 32", (1, 24, 8, 16, 3, 1, 1), (16, 3, 3, 24)),
    ("5x5 kernel", (1, 32, 8, 16, 5, 1, 2), (16, 5, 5, 32)),
    ("not tap-major", (1, 32, 8, 16, 3, 1, 1), (16, 32, 3, 3)),
    ("rows not padded to 32", (1, 3, 16, 16, 7, 2, 3), (16, 147)),
    ("rows for a 3x3 kernel", (1, 3, 16, 16, 3, 1, 1), (16, 32)),
])
def test_conv_packed_rejects(why, shape, wshape, hip, dmem, abi):
    from nnc_py_amd import runtime
    rng = np.random.default_rng(1)
    case = _packed_case(rng, *shape)
    case["tensors"]["w"] = np.zeros(wshape, np.float32)
    runtime.clear_error()
    out = caserun.run_case(hip, case, abi, dmem)["out"]
    assert runtime.last_error()[0] != 0, why
    assert not out.any()


def _gemm_case(rng, m, n, k, ta, tb, bias):
    a = rng.uniform(-1, 1, (k, m) if ta else (m, k)).astype(np.float32)
    b = rng.uniform(-1, 1, (n, k) if tb else (k, n)).astype(np.float32)
    tensors = {"a": a, "b": b, "out": np.zeros((m, n), np.float32)}
    if bias:
        tensors["c"] = rng.uniform(-1, 1, n).astype(np.float32)
    return {"name": f"gemm_{m}x{n}x{k}_t{ta}{tb}", "op": "nnc_gemm", "tensors": tensors,
            "args": [("t", "a"), ("t", "b"), ("t", "c") if bias else ("null",), ("t", "out"),
                     ("f", 1.0), ("f", 1.0), ("i", ta), ("i", tb)],
            "outputs": ["out"], "bar": "fp"}


GEMM_SHAPES = [
    (512, 512, 512, 0, 0, True),
    (384, 640, 1024, 0, 1, True),
    (256, 300, 777, 1, 0, False),
    (130, 250, 2048, 1, 1, True),
    (1024, 1024, 1024, 0, 0, True),
    (1, 1000, 512, 0, 1, True),     # ResNet FC at batch 1
    (32, 1000, 512, 0, 1, True),    # ResNet FC at batch 32
    # direct-to-LDS layouts: A x-contiguous (transA, M % 4 == 0) with B
    # x-contiguous and k-contiguous, and K tails that are whole 16-byte
    # chunks but not whole 32-k slices
    (256, 192, 100, 1, 0, True),
    (200, 128, 68, 0, 1, True),
    (64, 96, 40, 1, 1, False),
    (1536, 1536, 132, 0, 1, True),  # 128x128 direct-to-LDS tiles, K tail of 4
    # at most 32 rows, both operands k-contiguous: one launch, 16 columns per
    # workgroup, K over 8 waves - one row block, N not a multiple of 16, a K
    # tail inside a 16-wide chunk, fewer chunks than waves, K = 1024
    (8, 1000, 512, 0, 1, True),     # ResNet FC at batch 8
    (17, 333, 1020, 0, 1, False),
    (32, 50, 36, 0, 1, True),
    (3, 40, 1024, 0, 1, True),
    # products up to 1 GFLOP on fewer than 1024 workgroups run on gemm_ws_k
    # (32x32 tiles, waves splitting K; every layout above that is not skinny
    # or a dot/GEMV, except 1024^3 and 1536^2 x 132); these keep
    # the other kernels covered: register-staged tiles (A k-contiguous with
    # K % 4 != 0), direct-to-LDS 64x64 with a K tail of one 16-byte chunk,
    # and 128x128 with a K tail of 4
    (300, 200, 777, 0, 1, True),
    (1024, 1100, 996, 0, 1, True),
    (2048, 2048, 132, 0, 1, True),
    # gemm_ws_k: tiles split over 8 workgroups (K = 4096), a split tile with
    # M and N tails, x-contiguous operands on both sides with a split
    (256, 256, 4096, 0, 1, True),
    (100, 70, 3000, 0, 0, False),
    (96, 160, 2500, 1, 0, True),
    # one output row, B row-major (gemv_fin_k): 16 K splits finished in the
    # kernel, a column block past N (1000 = 15 x 64 + 40), 13 splits of 3
    # rows (fewer rows than row lanes), 8 splits over 128 column blocks, no
    # split (4688 column blocks); N % 4 != 0 keeps the two-launch path
    (1, 4096, 4096, 0, 0, True),
    (1, 1000, 512, 0, 0, True),
    (1, 260, 37, 0, 0, False),
    (1, 8192, 100, 0, 0, True),
    (1, 300000, 8, 0, 0, True),
    (1, 333, 100, 0, 0, True),
]


@pytest.mark.parametrize("shape", GEMM_SHAPES, ids=[str(s) for s in GEMM_SHAPES])
def test_gemm_layouts_and_streamk(shape, hip, dmem, abi, oracle_lib):
    case = _gemm_case(np.random.default_rng(3), *shape)
    print(f"case {case['name']}", flush=True)
    exp = caserun.run_case(oracle_lib, case, abi)["out"]
    got = caserun.run_case(hip, case, abi, dmem)["out"]
    _check(got, exp, case["name"])


@pytest.mark.parametrize("m,n,k", [(300, 200, 777), (256, 256, 4096), (37, 45, 64)])
@pytest.mark.parametrize("c_shape", ["row", "matrix"])
def test_gemm_short_product_c_and_scales(m, n, k, c_shape, hip, dmem, abi, oracle_lib):
    """alpha * A B + beta * C on the short-product kernel (gemm_ws_k: whole
    32x32 tiles, tiles split over 8 workgroups, M and N tails), C a row of N
    (C[j]) or a whole [M, N] matrix (C[i*N + j]), against the oracle."""
    rng = np.random.default_rng(29)
    case = _gemm_case(rng, m, n, k, 0, 1, True)
    if c_shape == "matrix":
        case["tensors"]["c"] = rng.uniform(-1, 1, (m, n)).astype(np.float32)
    case["args"][4] = ("f", 0.5)
    case["args"][5] = ("f", -2.0)
    case["name"] += f"_c{c_shape}"
    print(f"case {case['name']}", flush=True)
    exp = caserun.run_case(oracle_lib, case, abi)["out"]
    got = caserun.run_case(hip, case, abi, dmem)["out"]
    _check(got, exp, case["name"])


# Shapes whose split tiles are finished inside the kernel by the last of
# their workgroups (no fixup launch, checked): 64 channels 3x3 with a
# residual over 12 x 56x56 (direct-to-LDS 64x128 tiles, 294 tiles of 18
# slices on 768 workgroups, at most 4 contributors per tile; 16-byte
# finish) and 11 x 57x57 (images of an odd pixel count: the finish's
# per-element path), GEMM 1024x768x1024 (direct-to-LDS 64x64
# tiles at one workgroup per CU, 192 tiles of 32 slices) and 2048x1024x256
# (128x128 tiles, 128 tiles of 8 slices); the short-product kernels' tiles
# split over 8 workgroups (conv 512 channels 3x3 over 7x7, GEMM
# 256x256x4096); the GEMV's 16 K splits of each 64-column block (1 x 1000
# x 4096); and the stem's fused max pool at 10 x 224x224, whose 512
# ranges of two or three conv rows finish the pool rows they share with
# their neighbours in the kernel.
IN_KERNEL_FINISH_CASES = ["conv_b12_64c_56", "conv_b11_64c_57", "conv_ws_b1_512c_7", "gemm_1024x768x1024", "gemm_2048x1024x256",
                          "gemm_ws_256x256x4096", "gemv_1x1000x4096", "stem_pool_b10"]


@pytest.mark.parametrize("which", IN_KERNEL_FINISH_CASES)
def test_in_kernel_finish_alternating_inputs(which, hip, dmem, abi, oracle_lib):
    """Two inputs in turn, four calls: the partials and tile counters the
    previous call left in the library's scratch differ from this call's, so
    a partial read before its writer's stores were visible, or a counter
    not back at zero, shows up as a wrong tile. Each call matches the
    oracle, and calls on the same input match each other to the bit."""
    def make(seed):
        rng = np.random.default_rng(seed)
        if which == "conv_b12_64c_56":
            return _packed_case(rng, 12, 64, 56, 64, 3, 1, 1)
        if which == "conv_b11_64c_57":
            return _packed_case(rng, 11, 64, 57, 64, 3, 1, 1)
        if which == "conv_ws_b1_512c_7":
            return _packed_case(rng, 1, 512, 7, 512, 3, 1, 1)
        if which == "stem_pool_b10":
            return _conv_maxpool_case(rng, 10, 224, 224, 64, True)
        if which == "gemv_1x1000x4096":
            return _gemm_case(rng, 1, 1000, 4096, 0, 0, True)
        m, n, k = {"gemm_1024x768x1024": (1024, 768, 1024), "gemm_2048x1024x256": (2048, 1024, 256),
                   "gemm_ws_256x256x4096": (256, 256, 4096)}[which]
        return _gemm_case(rng, m, n, k, 0, 1, True)
    from nnc_py_amd import runtime
    cases = [make(41), make(42)]
    exp = [caserun.run_case(oracle_lib, c, abi)["out"] for c in cases]
    first = [None, None]
    for call in range(4):
        q = call % 2
        print(f"case {which} call {call} input {q}", flush=True)
        runtime.profile_reset()
        runtime.profile_enable(True)
        got = caserun.run_case(hip, cases[q], abi, dmem)["out"]
        launched = {r["name"] for r in runtime.profile_table()}
        runtime.profile_enable(False)
        # the case exercises the in-kernel finish only while its plan keeps
        # every shared tile within the finish's contributor limit
        assert not any("fixup" in name for name in launched), sorted(launched)
        _check(got, exp[q], f"{which} call {call}")
        if first[q] is None:
            first[q] = got
        else:
            assert np.array_equal(got, first[q]), f"{which} call {call}: differs from the first call on this input"


def test_batched_matmul_broadcast_b(hip, dmem, abi, oracle_lib):
    """[12,96,72] x [72,136]: B broadcast over the batch (batch stride 0 on
    the direct-to-LDS path), each batch against the oracle's 2-D product."""
    rng = np.random.default_rng(6)
    a = rng.uniform(-1, 1, (12, 96, 72)).astype(np.float32)
    b = rng.uniform(-1, 1, (72, 136)).astype(np.float32)
    case = {"name": "bmm_bcast", "op": "nnc_matmul",
            "tensors": {"a": a, "b": b, "out": np.zeros((12, 96, 136), np.float32)},
            "args": [("t", "a"), ("t", "b"), ("t", "out")], "outputs": ["out"], "bar": "fp"}
    got = caserun.run_case(hip, case, abi, dmem)["out"]
    for q in (0, 5, 11):
        c2 = {"name": "slice", "op": "nnc_matmul",
              "tensors": {"a": a[q].copy(), "b": b, "out": np.zeros((96, 136), np.float32)},
              "args": [("t", "a"), ("t", "b"), ("t", "out")], "outputs": ["out"], "bar": "fp"}
        _check(got[q], caserun.run_case(oracle_lib, c2, abi)["out"], f"batch {q}")


def test_batched_matmul_streamk(hip, dmem, abi, oracle_lib):
    """[64,128,64] x [64,64,128] (the GEMM sweep's batched MatMul): numpy
    semantics per batch, checked slice by slice against the oracle's 2-D path."""
    rng = np.random.default_rng(4)
    a = rng.uniform(-1, 1, (64, 128, 64)).astype(np.float32)
    b = rng.uniform(-1, 1, (64, 64, 128)).astype(np.float32)
    case = {"name": "bmm", "op": "nnc_matmul", "tensors": {"a": a, "b": b, "out": np.zeros((64, 128, 128), np.float32)},
            "args": [("t", "a"), ("t", "b"), ("t", "out")], "outputs": ["out"], "bar": "fp"}
    got = caserun.run_case(hip, case, abi, dmem)["out"]
    for q in (0, 17, 63):
        c2 = {"name": "slice", "op": "nnc_matmul",
              "tensors": {"a": a[q].copy(), "b": b[q].copy(), "out": np.zeros((128, 128), np.float32)},
              "args": [("t", "a"), ("t", "b"), ("t", "out")], "outputs": ["out"], "bar": "fp"}
        _check(got[q], caserun.run_case(oracle_lib, c2, abi)["out"], f"batch {q}")


def _maxpool_case(x, ho, wo, k=3, s=2, p=1):
    n, c = x.shape[:2]
    out = np.full((n, c, ho, wo), 7.0, np.float32)
    return {"name": f"maxpool_{'x'.join(map(str, x.shape))}_to_{ho}x{wo}", "op": "nnc_maxpool2d",
            "tensors": {"x": x, "out": out},
            "args": [("t", "x"), ("t", "out")] + [("i", v) for v in (k, k, s, s, p, p)],
            "outputs": ["out"], "bar": "exact"}


# (N, C, H, W, Ho, Wo): the ResNet stem pool, two column chunks (Wo > 64),
# odd H, and outputs past the natural size (clamped and empty windows)
MAXPOOL_SHAPES = [
    (2, 64, 112, 112, 56, 56),    # 896 waves of 8 rows: 2 rows per wave
    (8, 64, 112, 112, 56, 56),    # 3584 waves of 8 rows: 4 rows per wave
    (20, 64, 112, 112, 56, 56),   # 8 rows per wave
    (1, 3, 130, 130, 65, 65),
    (2, 5, 7, 8, 4, 4),
    (1, 2, 8, 8, 6, 6),
    (1, 1, 2, 2, 1, 1),
]


@pytest.mark.parametrize("shape", MAXPOOL_SHAPES, ids=[str(s) for s in MAXPOOL_SHAPES])
def test_maxpool_3x3s2_bit_exact(shape, hip, dmem, abi, oracle_lib):
    n, c, h, w, ho, wo = shape
    rng = np.random.default_rng(3)
    x = rng.standard_normal((n, c, h, w)).astype(np.float32)
    # the first-element rule: NaN first in a window stays, later NaN is
    # skipped; signed zeros keep the first one seen
    flat = x.reshape(-1)
    flat[rng.integers(0, flat.size, 8)] = np.nan
    x[0, 0, :2, :] = -0.0
    x[0, 0, 0, ::2] = 0.0
    case = _maxpool_case(x, ho, wo)
    print(f"case {case['name']}", flush=True)
    exp = caserun.run_case(oracle_lib, case, abi)["out"]
    got = caserun.run_case(hip, case, abi, dmem)["out"]
    assert caserun.same_bits(got, exp), f"{case['name']}: {np.sum(got.view(np.uint32) != exp.view(np.uint32))} differ"


# Row kernels past the grid cap (more than 16384 rows: each wave walks
# several rows, loading the next while it reduces the current), a row of
# the largest register-resident length (4096 floats, no prefetch), and rows
# that fill every lane exactly (1024 and 768 floats: the kernels without
# per-lane bounds tests), past the grid cap and below it
ROW_SHAPES = [(40000, 64), (20000, 260), (17, 4096), (20000, 1024), (333, 768), (70, 256)]


@pytest.mark.parametrize("shape", ROW_SHAPES, ids=[str(s) for s in ROW_SHAPES])
def test_row_kernels_many_rows(shape, hip, dmem, abi, oracle_lib):
    rows, dim = shape
    rng = np.random.default_rng(17)
    x = (rng.standard_normal((rows, dim)) * 3).astype(np.float32)
    cases = [
        {"name": "softmax", "op": "nnc_softmax", "tensors": {"x": x, "out": np.zeros_like(x)},
         "args": [("t", "x"), ("t", "out"), ("i", -1)], "outputs": ["out"], "bar": "fp"},
        {"name": "layernorm", "op": "nnc_layernorm",
         "tensors": {"x": x, "g": rng.standard_normal(dim).astype(np.float32),
                     "b": rng.standard_normal(dim).astype(np.float32), "out": np.zeros_like(x)},
         "args": [("t", "x"), ("t", "g"), ("t", "b"), ("t", "out"), ("i", -1), ("f", 1e-5)],
         "outputs": ["out"], "bar": "fp"},
        {"name": "reducemean", "op": "nnc_reducemean",
         "tensors": {"x": x, "out": np.zeros((rows, 1), np.float32)},
         "args": [("t", "x"), ("t", "out"), ("i", 1), ("i", 1)], "outputs": ["out"], "bar": "fp"},
    ]
    for case in cases:
        print(f"case {case['name']} {shape}", flush=True)
        exp = caserun.run_case(oracle_lib, case, abi)["out"]
        got = caserun.run_case(hip, case, abi, dmem)["out"]
        _check(got, exp, f"{case['name']} {shape}")


GAP_GEMM_SHAPES = [
    (1, 512, 7, 7, 1000, "o", 1.0, 1.0),    # ResNet-18 classifier, batch 1
    (32, 512, 7, 7, 1000, "o", 1.0, 1.0),   # batch 32
    (5, 100, 3, 5, 70, "no", 0.5, -2.0),    # image / class tails, [N][O] bias, alpha, beta
    (3, 40, 1, 1, 9, None, 1.0, 1.0),       # 1x1 planes, no bias
    (6, 1024, 5, 5, 130, "o", 1.0, 1.0),    # the most channels (four float4 per lane), several staging rounds
    (2, 300, 9, 9, 17, "o", 1.0, 1.0),      # channels not a multiple of 256
]


@pytest.mark.parametrize("shape", GAP_GEMM_SHAPES, ids=[str(s[:5]) for s in GAP_GEMM_SHAPES])
def test_gap_gemm_nt_bit_exact(shape, hip, dmem, abi, oracle_lib):
    """nnc_hip_gap_gemm_nt against the oracle's nnc_avgpool2d + nnc_gemm_nt:
    the same float means and exact products, the double sums in another
    order, so every output is within one float ulp of the oracle's (and
    within the 1e-4 / 1e-3 bar)."""
    n, c, h, w, o, bias, alpha, beta = shape
    rng = np.random.default_rng(n * 7 + c)
    tensors = {"x": rng.standard_normal((n, c, h, w)).astype(np.float32),
               "w": (rng.standard_normal((o, c)) / np.sqrt(c)).astype(np.float32),
               "out": np.zeros((n, o), np.float32)}
    if bias == "o":
        tensors["c"] = (rng.standard_normal(o) * 0.01).astype(np.float32)
    elif bias == "no":
        tensors["c"] = rng.standard_normal((n, o)).astype(np.float32)
    case = {"name": f"gap_gemm_{shape}", "op": "nnc_hip_gap_gemm_nt", "tensors": tensors,
            "args": [("t", "x"), ("t", "w"), ("t", "c") if bias else ("null",), ("t", "out"), ("f", alpha),
                     ("f", beta)], "outputs": ["out"]}
    print(f"case {case['name']}", flush=True)
    exp = caserun.run_case(oracle_lib, case, abi)["out"]
    got = caserun.run_case(hip, case, abi, dmem)["out"]
    from nnc_py_amd import runtime
    assert runtime.last_error()[0] == 0, runtime.last_error()[1]
    assert caserun.fp_violations(got, exp, 1e-4, 1e-3).size == 0
    ulp = np.spacing(np.abs(exp).astype(np.float32))
    assert (np.abs(got - exp) <= ulp).all(), f"max diff {np.abs(got - exp).max():.3g}"
    print(f"{(got != exp).sum()} of {got.size} outputs one ulp off", flush=True)


def test_gap_gemm_nt_rejections(hip, dmem, abi):
    from nnc_py_amd import runtime
    rng = np.random.default_rng(3)
    bad = {"x": rng.standard_normal((2, 8, 4, 4)).astype(np.float32),
           "w": rng.standard_normal((5, 7)).astype(np.float32),  # 7 columns for 8 channels
           "out": np.zeros((2, 5), np.float32)}
    runtime.clear_error()
    out = caserun.run_case(hip, {"name": "bad", "op": "nnc_hip_gap_gemm_nt", "tensors": bad,
                                 "args": [("t", "x"), ("t", "w"), ("null",), ("t", "out"), ("f", 1.0), ("f", 1.0)],
                                 "outputs": ["out"]}, abi, dmem)["out"]
    assert runtime.last_error()[0] == 1 and not out.any()
    runtime.clear_error()


def _conv_maxpool_case(rng, n, h, w, co=64, bias=True):
    """nnc_hip_conv_maxpool case: the packed RGB 7x7 / stride 2 / pad 3 stem
    ([Co][160] rows) with relu, into the 3x3 / stride 2 / pad 1 max pool."""
    wr = (rng.standard_normal((co, 3, 7, 7)) * np.sqrt(2.0 / 147)).astype(np.float32)
    rows = np.zeros((co, 160), np.float32)
    rows[:, :147] = wr.transpose(0, 2, 3, 1).reshape(co, 147)
    ho, wo = (h + 6 - 7) // 2 + 1, (w + 6 - 7) // 2 + 1
    tensors = {"x": rng.standard_normal((n, 3, h, w)).astype(np.float32), "w": rows,
               "out": np.zeros((n, co, ho // 2, wo // 2), np.float32)}
    if bias:
        tensors["b"] = (rng.standard_normal(co) * 0.1).astype(np.float32)
    return {"name": f"conv_maxpool_{n}x{h}x{w}_{co}", "op": "nnc_hip_conv_maxpool", "tensors": tensors,
            "args": [("t", "x"), ("t", "w"), ("t", "b") if bias else ("null",), ("t", "out")]
            + [("i", v) for v in (7, 7, 2, 2, 3, 3)], "outputs": ["out"]}


@pytest.mark.parametrize("n,h,w,co,bias", [(1, 224, 224, 64, True), (2, 64, 100, 64, True), (8, 224, 224, 64, True),
                                           (3, 32, 255, 40, False), (5, 224, 224, 64, True), (16, 64, 64, 40, False)])
def test_conv_maxpool_stem(n, h, w, co, bias, hip, dmem, abi, oracle_lib):
    """The stem streamed into its max pool against the oracle's packed conv
    + relu + nnc_maxpool2d: within the conv bar of the oracle's double sums
    (the max itself is exact). Covers one-row and two-row bands with their
    band-boundary fixup, a full 128-pixel row (w = 255), Co < 64; from 512
    conv rows on (5 x 224x224, 16 x 64x64) the row kernel's fused pool with
    ranges of two rows."""
    case = _conv_maxpool_case(np.random.default_rng(n + h + w), n, h, w, co, bias)
    print(f"case {case['name']}", flush=True)
    exp = caserun.run_case(oracle_lib, case, abi)["out"]
    got = caserun.run_case(hip, case, abi, dmem)["out"]
    from nnc_py_amd import runtime
    assert runtime.last_error()[0] == 0, runtime.last_error()[1]
    _check(got, exp, case["name"])
    assert (got >= 0).all()


@pytest.mark.parametrize("n", [8, 20])
def test_conv_stem_pool_matches_unfused_bits(n, hip, dmem, abi):
    """The row kernel's fused pool against the same GPU convolution
    (nnc_hip_conv_packed, the row kernel at these sizes) followed by
    nnc_maxpool2d: the same bits. 8 images: 448 ranges of two rows; 20
    images: ranges of four and five rows, so ranges start on odd rows too."""
    case = _conv_maxpool_case(np.random.default_rng(31 + n), n, 224, 224, 64, True)
    got = caserun.run_case(hip, case, abi, dmem)["out"]
    t = case["tensors"]
    conv = {"name": "conv", "op": "nnc_hip_conv_packed",
            "tensors": {"x": t["x"], "w": t["w"], "b": t["b"], "out": np.zeros((n, 64, 112, 112), np.float32)},
            "args": [("t", "x"), ("t", "w"), ("t", "b"), ("null",), ("t", "out")] + [("i", v) for v in (7, 7, 2, 2, 3, 3, 1)],
            "outputs": ["out"], "bar": "fp"}
    mid = caserun.run_case(hip, conv, abi, dmem)["out"]
    pool = {"name": "pool", "op": "nnc_maxpool2d", "tensors": {"x": mid, "out": np.zeros_like(got)},
            "args": [("t", "x"), ("t", "out")] + [("i", v) for v in (3, 3, 2, 2, 1, 1)], "outputs": ["out"],
            "bar": "exact"}
    exp = caserun.run_case(hip, pool, abi, dmem)["out"]
    from nnc_py_amd import runtime
    assert runtime.last_error()[0] == 0, runtime.last_error()[1]
    assert caserun.same_bits(got, exp)


def test_conv_maxpool_rejections(hip, dmem, abi):
    """Odd conv output sizes and conv rows over 128 pixels are refused
    before any launch; the output is untouched."""
    from nnc_py_amd import runtime
    for n, h, w in ((1, 37, 64), (1, 64, 270)):
        case = _conv_maxpool_case(np.random.default_rng(1), n, h, w)
        case["tensors"]["out"] = np.zeros_like(case["tensors"]["out"])
        runtime.clear_error()
        out = caserun.run_case(hip, case, abi, dmem)["out"]
        assert runtime.last_error()[0] == 4 and not out.any(), (h, w)
    runtime.clear_error()


@pytest.mark.parametrize("n", [4099, 1 << 20])
@pytest.mark.parametrize("prog", range(8))
def test_fused_eltwise_matches_op_by_op(prog, n, hip, dmem, abi, oracle_lib):
    """nnc_hip_fused_eltwise against the same program run as single GPU
    calls through temporaries (the same device arithmetic: bit for bit),
    and against the oracle within the fp bar (sigmoid and tanh use the
    device's expf / tanhf); 4099 elements take the scalar tail; the output
    written over an input gives the same bits."""
    from ew_cases import EW_PROGRAMS, ew_arrays, ew_case, ew_compose
    from nnc_py_amd import runtime
    n_in, steps = EW_PROGRAMS[prog]
    print(f"case fused_eltwise program {prog} n {n}", flush=True)
    xs = ew_arrays(n_in, n, 60 + prog)
    got = caserun.run_case(hip, ew_case(n_in, steps, xs), abi, dmem)["out"]
    assert runtime.last_error()[0] == 0, runtime.last_error()[1]
    assert caserun.same_bits(got, ew_compose(hip, abi, steps, xs, dmem))
    _check(got, caserun.run_case(oracle_lib, ew_case(n_in, steps, xs), abi)["out"], f"fused_eltwise {prog}")
    over = caserun.run_case(hip, ew_case(n_in, steps, xs, out_key="i0"), abi, dmem)["i0"]
    assert caserun.same_bits(over, got)


@pytest.mark.parametrize("prog", [0, 1, 4, 5, 6, 7])
def test_fused_eltwise_compiled_chain_matches_general_kernel(prog, hip, dmem, abi):
    """A chain with a kernel compiled for it against the same chain on the
    general kernel, which reads the steps at run time: the same program
    given one more (unused) input no longer matches the library's table.
    Same bits; the output large enough for streaming stores."""
    from ew_cases import EW_PROGRAMS, EW_SPECIALIZED, ew_arrays, ew_case
    from nnc_py_amd import runtime
    n_in, steps = EW_PROGRAMS[prog]
    assert prog in EW_SPECIALIZED
    n = (20 << 20) + 4
    print(f"case fused_eltwise compiled chain {prog} n {n}", flush=True)
    xs = ew_arrays(n_in + 1, n, 90 + prog)
    got = caserun.run_case(hip, ew_case(n_in, steps, xs[:n_in]), abi, dmem)["out"]
    assert runtime.last_error()[0] == 0, runtime.last_error()[1]
    general = caserun.run_case(hip, ew_case(n_in + 1, steps, xs), abi, dmem)["out"]
    assert runtime.last_error()[0] == 0, runtime.last_error()[1]
    assert caserun.same_bits(got, general)


def test_fused_eltwise_rejects_malformed_programs(hip, dmem, abi):
    """Input and step counts out of range, an unknown op, step 0 reading the
    running value, an operand past the inputs, an input shorter than the
    output and Clip without bounds are refused before any launch
    (NNC_HIP_EINVAL), an int32 input too (NNC_HIP_EUNSUPP); the output is
    untouched."""
    from ew_cases import ew_case
    from nnc_py_amd import runtime
    xs = [np.ones(64, np.float32), np.ones(64, np.float32)]

    def edit(case, **kw):
        args = list(case["args"])
        for i, v in kw.items():
            args[int(i[1:])] = v
        case["args"] = args
        return case

    bad = [
        ("no inputs", edit(ew_case(2, [("ADD", 0, 1)], xs), a1=("i", 0))),
        ("five inputs", edit(ew_case(2, [("ADD", 0, 1)], xs), a1=("i", 5))),
        ("no steps", edit(ew_case(2, [("ADD", 0, 1)], xs), a3=("i", 0))),
        ("nine steps", edit(ew_case(2, [("ADD", 0, 1)] * 9, xs), a3=("i", 9))),
        ("unknown op", edit(ew_case(2, [("ADD", 0, 1)], xs), a2=("i32", [10, 0, 1]))),
        ("step 0 reads acc", ew_case(2, [("ADD", -1, 1)], xs)),
        ("operand past the inputs", ew_case(2, [("ADD", 0, 2)], xs)),
        ("clip without bounds", edit(ew_case(1, [("CLIP", 0, 0, -1.0, 1.0)], xs[:1]), a4=("null",))),
    ]
    short = ew_case(2, [("ADD", 0, 1)], [xs[0], np.ones(63, np.float32)])
    short["tensors"]["out"] = np.zeros(64, np.float32)
    bad.append(("short input", short))
    bad.append(("int32 input", ew_case(2, [("ADD", 0, 1)], [xs[0], np.ones(64, np.int32)])))
    for why, case in bad:
        case["tensors"]["out"] = np.full_like(case["tensors"]["out"], 7.0)
        runtime.clear_error()
        out = caserun.run_case(hip, case, abi, dmem)["out"]
        # a malformed call is NNC_HIP_EINVAL (1), a non-float32 tensor NNC_HIP_EUNSUPP (4)
        assert runtime.last_error()[0] == (4 if why == "int32 input" else 1), (why, runtime.last_error())
        assert (out == 7.0).all(), why
    runtime.clear_error()


@pytest.mark.parametrize("rows,W,col0,view,perm", [(1024, 768, 0, (8, 128, 4, 64), (0, 2, 1, 3)),
                                                   (1024, 768, 256, (8, 128, 4, 64), (0, 2, 3, 1)),
                                                   (1024, 768, 512, (8, 128, 4, 64), (0, 2, 1, 3)),
                                                   (33, 10, 3, (33, 7), (1, 0))])
def test_transpose_slice_matches_numpy(rows, W, col0, view, perm, hip, dmem, abi):
    """nnc_hip_transpose_slice on the GPU: the QKV head split of the
    encoder at batch 8, sequence 128 (each of the three pieces) and a ragged
    2-D slice, equal to numpy's slice, reshape and transpose; columns past
    the row and an output of the wrong size are refused."""
    from nnc_py_amd import runtime
    width = int(np.prod(view)) // rows
    x = np.random.default_rng(8).standard_normal((rows, W)).astype(np.float32)
    want = np.ascontiguousarray(x[:, col0:col0 + width].reshape(view).transpose(perm))
    print(f"case transpose_slice rows {rows} W {W} col0 {col0} perm {perm}", flush=True)

    def case(c0, out):
        return {"name": "ts", "op": "nnc_hip_transpose_slice", "tensors": {"x": x, "out": out},
                "args": [("t", "x"), ("t", "out"), ("i64", list(perm)), ("i", len(perm)), ("i", c0), ("i", width)],
                "outputs": ["out"]}
    got = caserun.run_case(hip, case(col0, np.zeros_like(want)), abi, dmem)["out"]
    assert runtime.last_error()[0] == 0, runtime.last_error()[1]
    assert got.tobytes() == want.tobytes()
    for c0, out, code in ((W - width + 1, np.full_like(want, 7.0), 1), (col0, np.full(want.size - 1, 7.0, np.float32), 1),
                          (col0, np.full(want.shape, 7, np.int8), 4), (col0, np.full(want.shape, 7, np.int32), 4)):
        # past the row, one element short (NNC_HIP_EINVAL); 1-byte elements,
        # float32 -> int32 (NNC_HIP_EUNSUPP)
        runtime.clear_error()
        bad = caserun.run_case(hip, case(c0, out), abi, dmem)["out"]
        assert runtime.last_error()[0] == code and (bad == 7).all(), runtime.last_error()
    runtime.clear_error()


def test_transformer_fusions_match_oracle_at_encoder_shapes(hip, dmem, abi, oracle_lib):
    """The three O3 transformer entry points at the encoder's own shapes
    (batch 8, sequence 128, d_model 256, 4 heads) on the GPU against the
    oracle's compositions of pinned entry points: nnc_hip_scaled_softmax on
    the [8,4,128,128] scores divided by sqrt(64) (nnc_div then nnc_softmax,
    ops.c:82-224, 260-310), nnc_hip_add_layernorm on the [1024,256]
    residual stream (nnc_add then nnc_layernorm, ops.c:2095-2171) within
    the fp bar, and nnc_hip_transpose_slice for each of Q, K, V of the
    [1024,768] projection (the slice copied out, then nnc_transpose,
    ops.c:1531-1581) bit for bit."""
    rng = np.random.default_rng(12)
    scores = (rng.standard_normal((8, 4, 128, 128)) * 4).astype(np.float32)
    case = {"name": "ssm", "op": "nnc_hip_scaled_softmax",
            "tensors": {"x": scores, "d": np.array([8.0], np.float32), "out": np.zeros_like(scores)},
            "args": [("t", "x"), ("t", "d"), ("t", "out"), ("i", -1)], "outputs": ["out"]}
    print("case scaled_softmax [8,4,128,128] vs oracle", flush=True)
    _check(caserun.run_case(hip, case, abi, dmem)["out"], caserun.run_case(oracle_lib, case, abi)["out"],
           "scaled_softmax [8,4,128,128]")
    a, b = (rng.standard_normal((1024, 256)).astype(np.float32) for _ in range(2))
    g = (1 + 0.1 * rng.standard_normal(256)).astype(np.float32)
    bb = (0.1 * rng.standard_normal(256)).astype(np.float32)
    case = {"name": "addln", "op": "nnc_hip_add_layernorm",
            "tensors": {"a": a, "b": b, "g": g, "bb": bb, "out": np.zeros_like(a)},
            "args": [("t", "a"), ("t", "b"), ("t", "g"), ("t", "bb"), ("t", "out"), ("i", -1), ("f", 1e-5)],
            "outputs": ["out"]}
    print("case add_layernorm [1024,256] vs oracle", flush=True)
    _check(caserun.run_case(hip, case, abi, dmem)["out"], caserun.run_case(oracle_lib, case, abi)["out"],
           "add_layernorm [1024,256]")
    qkv = rng.standard_normal((1024, 768)).astype(np.float32)
    for col0, perm in ((0, (0, 2, 1, 3)), (256, (0, 2, 3, 1)), (512, (0, 2, 1, 3))):
        out = np.zeros((8, 4, 128, 64) if perm[-1] == 3 else (8, 4, 64, 128), np.float32)
        case = {"name": "ts", "op": "nnc_hip_transpose_slice", "tensors": {"x": qkv, "out": out},
                "args": [("t", "x"), ("t", "out"), ("i64", list(perm)), ("i", 4), ("i", col0), ("i", 256)],
                "outputs": ["out"]}
        print(f"case transpose_slice [1024,768] col0 {col0} vs oracle", flush=True)
        got = caserun.run_case(hip, case, abi, dmem)["out"]
        want = caserun.run_case(oracle_lib, case, abi)["out"]
        assert caserun.same_bits(got, want), f"transpose_slice col0 {col0}"
    dmem.release()


@pytest.mark.parametrize("shape,axis,d", [((8, 4, 128, 128), -1, 4.0), ((32, 2048), -1, -1.5),
                                         ((4, 4000), -1, 0.125), ((3, 6, 5), 1, 2.5), ((5, 1001), -1, 3.0)])
def test_scaled_softmax_matches_div_then_softmax(shape, axis, d, hip, dmem, abi):
    """nnc_hip_scaled_softmax against nnc_div then nnc_softmax on the GPU,
    bit for bit: the row kernel dividing on load (rows of 128, 2048 with a
    negative divisor, 4000), a strided axis and a row that is no multiple of
    4 (the quotient written, then the softmax over it in place); a divisor of
    two elements is refused."""
    from nnc_py_amd import runtime
    rng = np.random.default_rng(6)
    x = (3 * rng.standard_normal(shape)).astype(np.float32)
    dv = np.array([d], np.float32)
    print(f"case scaled_softmax {shape} axis {axis} d {d}", flush=True)
    args = [("t", "x"), ("t", "d"), ("t", "out"), ("i", axis)]
    got = caserun.run_case(hip, {"name": "ssm", "op": "nnc_hip_scaled_softmax",
                                 "tensors": {"x": x, "d": dv, "out": np.zeros_like(x)},
                                 "args": args, "outputs": ["out"]}, abi, dmem)["out"]
    assert runtime.last_error()[0] == 0, runtime.last_error()[1]
    q = caserun.run_case(hip, {"name": "div", "op": "nnc_div", "tensors": {"x": x, "d": dv, "q": np.zeros_like(x)},
                               "args": [("t", "x"), ("t", "d"), ("t", "q")], "outputs": ["q"]}, abi, dmem)["q"]
    want = caserun.run_case(hip, {"name": "sm", "op": "nnc_softmax", "tensors": {"q": q, "out": np.zeros_like(x)},
                                  "args": [("t", "q"), ("t", "out"), ("i", axis)], "outputs": ["out"]}, abi, dmem)["out"]
    assert caserun.same_bits(got, want)
    two = {"name": "two", "op": "nnc_hip_scaled_softmax",
           "tensors": {"x": x, "d": np.array([d, d], np.float32), "out": np.full_like(x, 7.0)},
           "args": args, "outputs": ["out"]}
    runtime.clear_error()
    out = caserun.run_case(hip, two, abi, dmem)["out"]
    assert runtime.last_error()[0] == 1 and (out == 7.0).all()
    runtime.clear_error()


@pytest.mark.parametrize("shape,axis", [((3, 5, 256), -1), ((64, 3072), -1), ((2, 6, 4, 3), 1), ((3, 1001), -1)])
def test_add_layernorm_matches_add_then_layernorm(shape, axis, hip, dmem, abi):
    """nnc_hip_add_layernorm against nnc_add then nnc_layernorm on the GPU,
    bit for bit: the row kernel with contiguous scale / bias (spans 256 and
    3072), a strided axis (inner 12), and a span that is no multiple of 4
    (the sum written, then the layernorm over it in place); a second addend
    of another size is refused."""
    from nnc_py_amd import runtime
    rng = np.random.default_rng(9)
    a, b = (rng.standard_normal(shape).astype(np.float32) for _ in range(2))
    n = shape[axis % len(shape)]
    g, bb = (1 + 0.1 * rng.standard_normal(n)).astype(np.float32), (0.1 * rng.standard_normal(n)).astype(np.float32)
    tail = [("t", "g"), ("t", "bb"), ("t", "out"), ("i", axis), ("f", 1e-5)]
    print(f"case add_layernorm {shape} axis {axis}", flush=True)
    got = caserun.run_case(hip, {"name": "addln", "op": "nnc_hip_add_layernorm",
                                 "tensors": {"a": a, "b": b, "g": g, "bb": bb, "out": np.zeros_like(a)},
                                 "args": [("t", "a"), ("t", "b")] + tail, "outputs": ["out"]}, abi, dmem)["out"]
    assert runtime.last_error()[0] == 0, runtime.last_error()[1]
    s = caserun.run_case(hip, {"name": "add", "op": "nnc_add", "tensors": {"a": a, "b": b, "s": np.zeros_like(a)},
                               "args": [("t", "a"), ("t", "b"), ("t", "s")], "outputs": ["s"]}, abi, dmem)["s"]
    want = caserun.run_case(hip, {"name": "ln", "op": "nnc_layernorm",
                                  "tensors": {"s": s, "g": g, "bb": bb, "out": np.zeros_like(a)},
                                  "args": [("t", "s")] + tail, "outputs": ["out"]}, abi, dmem)["out"]
    assert caserun.same_bits(got, want)
    short = {"name": "short", "op": "nnc_hip_add_layernorm",
             "tensors": {"a": a, "b": b.ravel()[:-4].copy(), "g": g, "bb": bb, "out": np.full_like(a, 7.0)},
             "args": [("t", "a"), ("t", "b")] + tail, "outputs": ["out"]}
    runtime.clear_error()
    out = caserun.run_case(hip, short, abi, dmem)["out"]
    assert runtime.last_error()[0] == 1 and (out == 7.0).all()
    runtime.clear_error()


ATTENTION_SHAPES = [
    (8, 128, 4, 64, (0, 256, 512), 8.0, 0),     # the encoder: batch 8, sequence 128, 4 heads of 64
    (2, 32, 2, 32, (0, 64, 128), 5.65, 0),      # one key wave, heads of 32 (four key groups)
    (3, 96, 1, 64, (128, 0, 64), -1.5, 4),      # keys past 96 masked, Q after K and V, a wider row
    (1, 64, 3, 32, (0, 96, 192), 2.0, 0),
    (2, 32, 2, 64, (0, 128, 256), 8.0, 0),      # heads of 64 over 32 keys: the second key chunk masked
    (1, 64, 8, 64, (0, 512, 1024), 8.0, 0),     # eight heads of 64, half the keys masked
]


@pytest.mark.parametrize("shape", ATTENTION_SHAPES, ids=[str(s[:4]) for s in ATTENTION_SHAPES])
def test_attention_matches_oracle(shape, hip, dmem, abi, oracle_lib):
    """nnc_hip_attention on the GPU against the oracle's composition (per
    batch and head: Q K^T, the division, the softmax, the product with V,
    heads merged) within the fp bar, and the same bits on a second run."""
    from test_oracle import attention_case
    batch, seq, heads, dh, cols, d, extra = shape
    case = attention_case(np.random.default_rng(47), batch, seq, heads, dh, cols, d, extra)
    print(f"case attention {shape}", flush=True)
    got = caserun.run_case(hip, case, abi, dmem)["out"]
    from nnc_py_amd import runtime
    assert runtime.last_error()[0] == 0, runtime.last_error()[1]
    _check(got, caserun.run_case(oracle_lib, case, abi)["out"], f"attention {shape}")
    assert caserun.same_bits(caserun.run_case(hip, case, abi, dmem)["out"], got)


def test_attention_rejects(hip, dmem, abi):
    """Refused before any launch, the output untouched: a sequence that is
    no multiple of 32 or longer than 128, a head of 48, a column offset
    that is no multiple of 4 floats, columns past the row, a two-element
    divisor, an output of the wrong size, int32 qkv."""
    from nnc_py_amd import runtime
    from test_oracle import attention_case

    def variant(seq=64, dh=32, cols=(0, 64, 128), div=None, out=None, qkv_dtype=None):
        c = attention_case(np.random.default_rng(1), 1, seq, 2, dh, cols, 2.0, extra=8)
        if div is not None:
            c["tensors"]["d"] = div
        if out is not None:
            c["tensors"]["out"] = out
        if qkv_dtype is not None:
            c["tensors"]["qkv"] = c["tensors"]["qkv"].astype(qkv_dtype)
        c["tensors"]["out"] = np.full_like(c["tensors"]["out"], 7.0)
        return c
    bad = [("seq 100", variant(seq=100), 4), ("seq 160", variant(seq=160), 4), ("head 48", variant(dh=48), 4),
           ("column 2", variant(cols=(2, 64, 128)), 4), ("past the row", variant(cols=(0, 64, 140)), 1),
           ("two-element divisor", variant(div=np.array([2.0, 2.0], np.float32)), 1),
           ("short output", variant(out=np.zeros((63, 64), np.float32)), 1),
           ("int32 qkv", variant(qkv_dtype=np.int32), 4)]
    for why, c, code in bad:
        runtime.clear_error()
        out = caserun.run_case(hip, c, abi, dmem)["out"]
        assert runtime.last_error()[0] == code, (why, runtime.last_error())
        assert (out == 7.0).all(), why
    runtime.clear_error()
