"""Pin the CPU oracle (oracle/nnc_oracle.c).

1. Bit-for-bit against the golden vectors, which the reference runtime itself
   produced (tests/golden/make_golden.py).
2. Bit-for-bit against the reference runtime on fresh random cases, where
   oracle/_ref is built.
3. Against closed forms that a plausible restatement mistake (dropped term,
   swapped index, transposed operand, wrong pad side) would break.
"""

from __future__ import annotations

import numpy as np
import pytest

import caserun
from conftest import GOLDEN

F32 = np.float32


@pytest.mark.parametrize("case", GOLDEN, ids=[c["name"] for c in GOLDEN])
def test_oracle_matches_reference_golden(case, oracle_lib, abi):
    got = caserun.run_case(oracle_lib, case, abi)
    for key, exp in case["expected"].items():
        assert caserun.same_bits(got[key], exp), f"{case['name']}:{key} differs from reference"


# ---------------------------------------------------------------------------
# fresh random cases, oracle vs reference (bit-exact)
# ---------------------------------------------------------------------------
def _conv_case(rng, op, n, ci, h, w, co, kh, kw, sh, sw, ph, pw, bias=True):
    ho = (h + 2 * ph - kh) // sh + 1
    wo = (w + 2 * pw - kw) // sw + 1
    t = {"x": rng.standard_normal((n, ci, h, w)).astype(F32),
         "w": rng.standard_normal((co, ci, kh, kw)).astype(F32),
         "out": np.zeros((n, co, ho, wo), F32)}
    args = [("t", "x"), ("t", "w")]
    if bias:
        t["b"] = rng.standard_normal((co,)).astype(F32)
        args.append(("t", "b"))
    else:
        args.append(("null",))
    args += [("t", "out"), ("i", kh), ("i", kw), ("i", sh), ("i", sw), ("i", ph), ("i", pw)]
    return {"name": "rand", "op": op, "tensors": t, "args": args, "outputs": ["out"]}


@pytest.mark.parametrize("seed", range(6))
def test_oracle_conv_random_vs_reference(seed, oracle_lib, ref_lib, abi):
    rng = np.random.default_rng(1000 + seed)
    kh = int(rng.integers(1, 6))
    kw = int(rng.integers(1, 6))
    sh, sw = int(rng.integers(1, 3)), int(rng.integers(1, 3))
    ph, pw = int(rng.integers(0, kh)), int(rng.integers(0, kw))
    c = _conv_case(rng, ["nnc_conv", "nnc_conv_relu", "nnc_conv_sigmoid"][seed % 3],
                   int(rng.integers(1, 3)), int(rng.integers(1, 5)), int(rng.integers(kh, 12)),
                   int(rng.integers(kw, 12)), int(rng.integers(1, 6)), kh, kw, sh, sw, ph, pw,
                   bias=bool(seed % 2))
    a = caserun.run_case(oracle_lib, c, abi)["out"]
    b = caserun.run_case(ref_lib, c, abi)["out"]
    assert caserun.same_bits(a, b)


@pytest.mark.parametrize("shape", [(56, 56), (28, 28), (7, 7), (3, 3), (2, 9)])
def test_oracle_conv3x3_fast_paths_vs_reference(shape, oracle_lib, ref_lib, abi):
    """The reference 3x3 s1/s2 paths use SSE2 interiors and border fallbacks;
    the oracle's single loop must agree with every one of them."""
    rng = np.random.default_rng(sum(shape))
    for op, s in (("nnc_conv", 1), ("nnc_conv", 2), ("nnc_conv_relu", 1)):
        c = _conv_case(rng, op, 1, 3, shape[0], shape[1], 4, 3, 3, s, s, 1, 1)
        assert caserun.same_bits(caserun.run_case(oracle_lib, c, abi)["out"],
                                 caserun.run_case(ref_lib, c, abi)["out"])
    c = _conv_case(rng, "nnc_conv7x7_s2", 1, 3, shape[0] + 6, shape[1] + 6, 2, 7, 7, 2, 2, 3, 3)
    c["args"] = c["args"][:4]
    assert caserun.same_bits(caserun.run_case(oracle_lib, c, abi)["out"],
                             caserun.run_case(ref_lib, c, abi)["out"])


@pytest.mark.parametrize("seed", range(4))
def test_oracle_matmul_gemm_random_vs_reference(seed, oracle_lib, ref_lib, abi):
    rng = np.random.default_rng(2000 + seed)
    M, K, N = (int(v) for v in rng.integers(1, 40, 3))
    mm = {"name": "mm", "op": "nnc_matmul",
          "tensors": {"a": rng.standard_normal((M, K)).astype(F32),
                      "b": rng.standard_normal((K, N)).astype(F32), "out": np.zeros((M, N), F32)},
          "args": [("t", "a"), ("t", "b"), ("t", "out")], "outputs": ["out"]}
    assert caserun.same_bits(caserun.run_case(oracle_lib, mm, abi)["out"],
                             caserun.run_case(ref_lib, mm, abi)["out"])
    ta, tb = seed % 2, seed // 2
    g = {"name": "g", "op": "nnc_gemm",
         "tensors": {"a": rng.standard_normal((K, M) if ta else (M, K)).astype(F32),
                     "b": rng.standard_normal((N, K) if tb else (K, N)).astype(F32),
                     "c": rng.standard_normal((M, N)).astype(F32), "out": np.zeros((M, N), F32)},
         "args": [("t", "a"), ("t", "b"), ("t", "c"), ("t", "out"), ("f", 0.75), ("f", -1.5),
                  ("i", ta), ("i", tb)], "outputs": ["out"]}
    assert caserun.same_bits(caserun.run_case(oracle_lib, g, abi)["out"],
                             caserun.run_case(ref_lib, g, abi)["out"])


@pytest.mark.parametrize("seed", range(4))
def test_oracle_rowwise_random_vs_reference(seed, oracle_lib, ref_lib, abi):
    rng = np.random.default_rng(3000 + seed)
    shape = tuple(int(v) for v in rng.integers(1, 9, 3))
    axis = int(rng.integers(-3, 3))
    x = (rng.standard_normal(shape) * 4).astype(F32)
    red_shape = list(shape)
    red_shape[axis] = 1
    for op, t, args in [
        ("nnc_softmax", {"x": x, "out": np.zeros_like(x)}, [("t", "x"), ("t", "out"), ("i", axis)]),
        ("nnc_reducesum", {"x": x, "out": np.zeros(red_shape, F32)},
         [("t", "x"), ("t", "out"), ("i", axis), ("i", 1)]),
        ("nnc_reducemean", {"x": x, "out": np.zeros(red_shape, F32)},
         [("t", "x"), ("t", "out"), ("i", axis), ("i", 0)]),
        ("nnc_layernorm", {"x": x, "g": rng.standard_normal(shape[axis]).astype(F32),
                           "b": rng.standard_normal(shape[axis]).astype(F32), "out": np.zeros_like(x)},
         [("t", "x"), ("t", "g"), ("t", "b"), ("t", "out"), ("i", axis), ("f", 1e-5)]),
    ]:
        c = {"name": op, "op": op, "tensors": t, "args": args, "outputs": ["out"]}
        assert caserun.same_bits(caserun.run_case(oracle_lib, c, abi)["out"],
                                 caserun.run_case(ref_lib, c, abi)["out"]), op


# ---------------------------------------------------------------------------
# closed forms (no reference needed)
# ---------------------------------------------------------------------------
def _np_conv_f64(x, w, b, sh, sw, ph, pw, ho, wo):
    """float64 direct convolution with top/left padding; fp32 products are exact
    in float64, so rounding the float64 sum once reproduces a float64
    accumulator up to summation order (within 1 ulp for these sizes)."""
    n, ci, h, ww = x.shape
    co, _, kh, kw = w.shape
    pad = np.zeros((n, ci, max(h + 2 * ph, (ho - 1) * sh + kh) + kh, max(ww + 2 * pw, (wo - 1) * sw + kw) + kw))
    pad[:, :, ph:ph + h, pw:pw + ww] = x
    out = np.zeros((n, co, ho, wo))
    for r in range(kh):
        for c in range(kw):
            patch = pad[:, :, r:r + (ho - 1) * sh + 1:sh, c:c + (wo - 1) * sw + 1:sw]
            out += np.einsum("nchw,oc->nohw", patch, w[:, :, r, c].astype(np.float64))
    if b is not None:
        out += b.astype(np.float64)[None, :, None, None]
    return out


@pytest.mark.parametrize("spec", [(3, 3, 1, 1, 1, 1), (3, 3, 2, 2, 1, 1), (1, 1, 2, 2, 0, 0),
                                  (7, 7, 2, 2, 3, 3), (5, 5, 1, 1, 2, 2), (3, 5, 2, 1, 1, 2)])
def test_oracle_conv_closed_form(spec, oracle_lib, abi):
    kh, kw, sh, sw, ph, pw = spec
    rng = np.random.default_rng(kh * 100 + kw)
    c = _conv_case(rng, "nnc_conv", 2, 3, 11, 10, 5, kh, kw, sh, sw, ph, pw)
    got = caserun.run_case(oracle_lib, c, abi)["out"]
    t = c["tensors"]
    ref = _np_conv_f64(t["x"], t["w"], t["b"], sh, sw, ph, pw, got.shape[2], got.shape[3])
    np.testing.assert_allclose(got, ref.astype(F32), rtol=2e-7, atol=1e-6)


def test_oracle_conv_pad_only_top_left(oracle_lib, abi):
    """Output extent decides the bottom/right padding (c_emitter.py:1051-1058):
    an output one row shorter than 'same' must equal the same-pad result
    cropped, not a shifted window."""
    rng = np.random.default_rng(5)
    c = _conv_case(rng, "nnc_conv", 1, 2, 6, 6, 3, 3, 3, 1, 1, 1, 1)
    full = caserun.run_case(oracle_lib, c, abi)["out"]
    c2 = dict(c)
    c2["tensors"] = dict(c["tensors"], out=np.zeros((1, 3, 5, 5), F32))
    crop = caserun.run_case(oracle_lib, c2, abi)["out"]
    assert caserun.same_bits(crop, full[:, :, :5, :5].copy())


def test_oracle_gemm_closed_form(oracle_lib, abi):
    rng = np.random.default_rng(9)
    for ta in (0, 1):
        for tb in (0, 1):
            M, K, N = 7, 13, 5
            a = rng.uniform(-1, 1, (K, M) if ta else (M, K)).astype(F32)
            b = rng.uniform(-1, 1, (N, K) if tb else (K, N)).astype(F32)
            cvec = rng.uniform(-1, 1, (N,)).astype(F32)
            c = {"name": "g", "op": "nnc_gemm",
                 "tensors": {"a": a, "b": b, "c": cvec, "out": np.zeros((M, N), F32)},
                 "args": [("t", "a"), ("t", "b"), ("t", "c"), ("t", "out"), ("f", 2.0), ("f", 0.5),
                          ("i", ta), ("i", tb)], "outputs": ["out"]}
            got = caserun.run_case(oracle_lib, c, abi)["out"]
            A = (a.T if ta else a).astype(np.float64)
            B = (b.T if tb else b).astype(np.float64)
            ref = (2.0 * (A @ B) + 0.5 * cvec.astype(np.float64)).astype(F32)
            np.testing.assert_allclose(got, ref, rtol=1e-6, atol=1e-6)


def test_oracle_matmul_batched_reproduces_reference_stepping(oracle_lib, abi):
    """The reference advances A and B by their batch COUNT per batch
    (ops.c:1687-1704); batch 0 is a true product, later batches are shifted
    windows. The oracle must show exactly that."""
    rng = np.random.default_rng(12)
    a = rng.standard_normal((3, 4, 5)).astype(F32)
    b = rng.standard_normal((3, 5, 6)).astype(F32)
    c = {"name": "bm", "op": "nnc_matmul",
         "tensors": {"a": a, "b": b, "out": np.zeros((3, 4, 6), F32)},
         "args": [("t", "a"), ("t", "b"), ("t", "out")], "outputs": ["out"]}
    got = caserun.run_case(oracle_lib, c, abi)["out"]
    np.testing.assert_allclose(got[0], a[0] @ b[0], rtol=1e-5, atol=1e-5)
    fa, fb = a.ravel(), b.ravel()
    a1 = fa[3:3 + 20].reshape(4, 5)
    b1 = fb[3:3 + 30].reshape(5, 6)
    np.testing.assert_allclose(got[1], a1 @ b1, rtol=1e-5, atol=1e-5)


def test_oracle_softmax_and_layernorm_invariants(oracle_lib, abi):
    rng = np.random.default_rng(3)
    x = (rng.standard_normal((16, 100)) * 5).astype(F32)
    c = {"name": "s", "op": "nnc_softmax", "tensors": {"x": x, "out": np.zeros_like(x)},
         "args": [("t", "x"), ("t", "out"), ("i", -1)], "outputs": ["out"]}
    p = caserun.run_case(oracle_lib, c, abi)["out"].astype(np.float64)
    np.testing.assert_allclose(p.sum(1), 1.0, atol=1e-5)
    e = np.exp(x.astype(np.float64) - x.max(1, keepdims=True))
    np.testing.assert_allclose(p, e / e.sum(1, keepdims=True), rtol=1e-5, atol=1e-7)
    g = rng.standard_normal(100).astype(F32)
    bb = rng.standard_normal(100).astype(F32)
    c = {"name": "l", "op": "nnc_layernorm",
         "tensors": {"x": x, "g": g, "b": bb, "out": np.zeros_like(x)},
         "args": [("t", "x"), ("t", "g"), ("t", "b"), ("t", "out"), ("i", -1), ("f", 1e-5)],
         "outputs": ["out"]}
    y = caserun.run_case(oracle_lib, c, abi)["out"].astype(np.float64)
    xd = x.astype(np.float64)
    ref = (xd - xd.mean(1, keepdims=True)) / np.sqrt(xd.var(1, keepdims=True) + 1e-5) * g + bb
    np.testing.assert_allclose(y, ref, rtol=1e-4, atol=1e-4)


def test_oracle_pools_and_copies_closed_form(oracle_lib, abi):
    rng = np.random.default_rng(4)
    x = rng.standard_normal((2, 3, 9, 8)).astype(F32)
    c = {"name": "mp", "op": "nnc_maxpool2d",
         "tensors": {"x": x, "out": np.zeros((2, 3, 5, 4), F32)},
         "args": [("t", "x"), ("t", "out"), ("i", 3), ("i", 3), ("i", 2), ("i", 2), ("i", 1), ("i", 1)],
         "outputs": ["out"]}
    got = caserun.run_case(oracle_lib, c, abi)["out"]
    pad = np.full((2, 3, 12, 11), -np.inf, F32)
    pad[:, :, 1:10, 1:9] = x
    ref = np.stack([np.stack([pad[:, :, 2 * i:2 * i + 3, 2 * j:2 * j + 3].max((2, 3)) for j in range(4)], -1)
                    for i in range(5)], -2)
    assert caserun.same_bits(got, ref.astype(F32))
    c = {"name": "ap", "op": "nnc_avgpool2d",
         "tensors": {"x": x, "out": np.zeros((2, 3, 1, 1), F32)},
         "args": [("t", "x"), ("t", "out"), ("i", 9), ("i", 8), ("i", 9), ("i", 8), ("i", 0), ("i", 0)],
         "outputs": ["out"]}
    got = caserun.run_case(oracle_lib, c, abi)["out"]
    np.testing.assert_allclose(got[..., 0, 0], x.astype(np.float64).mean((2, 3)), rtol=1e-5, atol=1e-6)
    perm = (0, 2, 3, 1)
    c = {"name": "tr", "op": "nnc_transpose",
         "tensors": {"x": x, "out": np.zeros(tuple(x.shape[p] for p in perm), F32)},
         "args": [("t", "x"), ("t", "out"), ("i64", list(perm)), ("i", 4)], "outputs": ["out"]}
    assert caserun.same_bits(caserun.run_case(oracle_lib, c, abi)["out"], np.transpose(x, perm).copy())
    parts = [rng.standard_normal((2, k, 3)).astype(F32) for k in (1, 4, 2)]
    t = {f"p{i}": p for i, p in enumerate(parts)}
    t["out"] = np.zeros((2, 7, 3), F32)
    c = {"name": "cc", "op": "nnc_concat", "tensors": t,
         "args": [("tl", ["p0", "p1", "p2"]), ("t", "out"), ("i", 3), ("i", 1)], "outputs": ["out"]}
    assert caserun.same_bits(caserun.run_case(oracle_lib, c, abi)["out"], np.concatenate(parts, 1))


def test_oracle_binary_flat_modulo_rule(oracle_lib, abi):
    a = np.arange(8, dtype=F32).reshape(2, 4)
    b = np.array([10.0, 20.0], F32)
    c = {"name": "fm", "op": "nnc_add", "tensors": {"a": a, "b": b, "out": np.zeros_like(a)},
         "args": [("t", "a"), ("t", "b"), ("t", "out")], "outputs": ["out"]}
    got = caserun.run_case(oracle_lib, c, abi)["out"].ravel()
    assert got.tolist() == [10, 21, 12, 23, 14, 25, 16, 27]  # b[i % 2], not numpy's rule
    c["tensors"] = {"a": np.arange(3, dtype=F32), "b": np.arange(5, dtype=F32),
                    "out": np.full(8, -1.0, F32)}
    got = caserun.run_case(oracle_lib, c, abi)["out"]
    assert got.tolist() == [0, 2, 4, -1, -1, -1, -1, -1]  # only min(3,5,8) written


# ---------------------------------------------------------------------------
# the mi355x target's entry points that have no reference counterpart are
# compositions of pinned ones; check the composition against numpy so that a
# wrong unpacking index, a dropped residual or a wrong activation fails
# ---------------------------------------------------------------------------
def _relu(x):
    return np.where(x > 0, x, F32(0)).astype(F32)


@pytest.mark.parametrize("act", [0, 1, 2])
@pytest.mark.parametrize("res", [False, True])
@pytest.mark.parametrize("kernel", [(3, 3, 1, 1, 1, 1), (3, 3, 2, 2, 1, 1), (1, 1, 2, 2, 0, 0)])
def test_oracle_conv_packed_composition(act, res, kernel, oracle_lib, abi):
    kh, kw, sh, sw, ph, pw = kernel
    rng = np.random.default_rng(31 + act + 3 * res)
    c = _conv_case(rng, "nnc_conv", 2, 32, 9, 9, 6, kh, kw, sh, sw, ph, pw)
    conv = caserun.run_case(oracle_lib, c, abi)["out"]
    t = dict(c["tensors"])
    t["w"] = np.ascontiguousarray(t["w"].transpose(0, 2, 3, 1))
    args = c["args"][:3] + [("t", "res") if res else ("null",)] + c["args"][3:] + [("i", act)]
    t["res"] = rng.standard_normal(conv.shape).astype(F32)
    got = caserun.run_case(oracle_lib, {"name": "packed", "op": "nnc_hip_conv_packed", "tensors": t,
                                        "args": args, "outputs": ["out"]}, abi)["out"]
    pre = (conv + t["res"]).astype(F32) if res else conv
    if act == 0:
        assert caserun.same_bits(got, pre)
    elif act == 1:
        assert caserun.same_bits(got, _relu(pre))
    else:
        np.testing.assert_allclose(got, 1.0 / (1.0 + np.exp(-pre.astype(np.float64))), rtol=1e-6, atol=1e-7)
    # and the unpacked weights give the float64 convolution
    ref = _np_conv_f64(c["tensors"]["x"], c["tensors"]["w"], c["tensors"]["b"], sh, sw, ph, pw,
                       conv.shape[2], conv.shape[3])
    np.testing.assert_allclose(conv, ref.astype(F32), rtol=2e-7, atol=1e-5)


def test_oracle_conv_packed_rows_stem(oracle_lib, abi):
    """[Co][Kp] packing (3-channel 7x7 stem): rows of tap-major weights with
    zeros past K give the reference convolution."""
    rng = np.random.default_rng(37)
    c = _conv_case(rng, "nnc_conv_relu", 2, 3, 23, 23, 5, 7, 7, 2, 2, 3, 3)
    ref = caserun.run_case(oracle_lib, c, abi)["out"]
    t = dict(c["tensors"])
    w = t["w"]
    rows = np.zeros((w.shape[0], 160), F32)
    rows[:, :147] = w.transpose(0, 2, 3, 1).reshape(w.shape[0], 147)
    rows[:, 147:] = 1e30  # padding is ignored
    t["w"] = rows
    args = c["args"][:3] + [("null",)] + c["args"][3:] + [("i", 1)]
    got = caserun.run_case(oracle_lib, {"name": "stem", "op": "nnc_hip_conv_packed", "tensors": t, "args": args,
                                        "outputs": ["out"]}, abi)["out"]
    assert caserun.same_bits(got, ref)


@pytest.mark.parametrize("act", [0, 1, 2])
@pytest.mark.parametrize("ps,xh", [(2, 12), (1, 6), (2, 13)])
def test_oracle_conv_proj_composition(act, ps, xh, oracle_lib, abi):
    """nnc_hip_conv_proj: rows [W3 tap-major | Wp] give the float64 3x3
    convolution of x plus the float64 strided 1x1 convolution of p plus
    the bias, then the activation; a row split one column off, a missed
    stride or a dropped projection fails."""
    rng = np.random.default_rng(43 + act)
    n, ci, h, co, cx = 2, 32, 6, 5, 32
    x = rng.standard_normal((n, ci, h, h)).astype(F32)
    p = rng.standard_normal((n, cx, xh, xh)).astype(F32)
    w3 = rng.standard_normal((co, ci, 3, 3)).astype(F32)
    w1 = rng.standard_normal((co, cx, 1, 1)).astype(F32)
    b = rng.standard_normal(co).astype(F32)
    rows = np.concatenate([w3.transpose(0, 2, 3, 1).reshape(co, -1), w1.reshape(co, cx)], axis=1)
    t = {"x": x, "w": np.ascontiguousarray(rows), "b": b, "p": p, "out": np.zeros((n, co, h, h), F32)}
    args = [("t", "x"), ("t", "w"), ("t", "b"), ("t", "p"), ("t", "out")]
    args += [("i", v) for v in (3, 3, 1, 1, 1, 1, ps, ps, act)]
    got = caserun.run_case(oracle_lib, {"name": "proj", "op": "nnc_hip_conv_proj", "tensors": t, "args": args,
                                        "outputs": ["out"]}, abi)["out"]
    pre = (_np_conv_f64(x, w3, b, 1, 1, 1, 1, h, h)
           + _np_conv_f64(p, w1, np.zeros(co, F32), ps, ps, 0, 0, h, h))
    if act == 1:
        want = np.maximum(pre, 0.0)
    elif act == 2:
        want = 1.0 / (1.0 + np.exp(-pre))
    else:
        want = pre
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-5)


def test_oracle_conv_add_relu_composition(oracle_lib, abi):
    rng = np.random.default_rng(41)
    c = _conv_case(rng, "nnc_conv", 2, 5, 8, 8, 4, 3, 3, 1, 1, 1, 1)
    conv = caserun.run_case(oracle_lib, c, abi)["out"]
    t = dict(c["tensors"], res=rng.standard_normal(conv.shape).astype(F32))
    args = c["args"][:3] + [("t", "res")] + c["args"][3:]
    got = caserun.run_case(oracle_lib, {"name": "car", "op": "nnc_hip_conv_add_relu", "tensors": t,
                                        "args": args, "outputs": ["out"]}, abi)["out"]
    assert caserun.same_bits(got, _relu((conv + t["res"]).astype(F32)))


@pytest.mark.parametrize("bias_shape", [None, (7,), (5, 7)])
def test_oracle_matmul_relu_composition(bias_shape, oracle_lib, abi):
    rng = np.random.default_rng(43)
    a = rng.standard_normal((5, 6)).astype(F32)
    b = rng.standard_normal((6, 7)).astype(F32)
    t = {"a": a, "b": b, "out": np.zeros((5, 7), F32)}
    mm = caserun.run_case(oracle_lib, {"name": "mm", "op": "nnc_matmul", "tensors": dict(t),
                                       "args": [("t", "a"), ("t", "b"), ("t", "out")], "outputs": ["out"]},
                          abi)["out"]
    np.testing.assert_allclose(mm, a.astype(np.float64) @ b, rtol=1e-5, atol=1e-5)
    args = [("t", "a"), ("t", "b"), ("null",), ("t", "out")]
    want = mm
    if bias_shape:
        t["bias"] = rng.standard_normal(bias_shape).astype(F32)
        args[2] = ("t", "bias")
        want = (mm + t["bias"]).astype(F32)
    got = caserun.run_case(oracle_lib, {"name": "mmr", "op": "nnc_matmul_relu", "tensors": t, "args": args,
                                        "outputs": ["out"]}, abi)["out"]
    assert caserun.same_bits(got, _relu(want))


@pytest.mark.parametrize("n,c,h,w,o,bias", [(2, 16, 7, 7, 10, "o"), (3, 5, 3, 4, 7, "no"), (1, 8, 1, 1, 3, None)])
def test_oracle_gap_gemm_nt_composition(n, c, h, w, o, bias, oracle_lib, abi):
    """nnc_hip_gap_gemm_nt: the plane means are the sequential float sums
    (numpy cumsum is sequential) divided by H*W, bit for bit; the outputs
    the float64 dot products with w, times alpha, plus beta * c, rounded to
    float."""
    rng = np.random.default_rng(41 + c)
    x = rng.standard_normal((n, c, h, w)).astype(F32)
    wt = rng.standard_normal((o, c)).astype(F32)
    tensors = {"x": x, "w": wt, "out": np.zeros((n, o), F32)}
    args = [("t", "x"), ("t", "w")]
    if bias == "o":
        tensors["c"] = rng.standard_normal(o).astype(F32)
    elif bias == "no":
        tensors["c"] = rng.standard_normal((n, o)).astype(F32)
    args += [("t", "c") if bias else ("null",), ("t", "out"), ("f", 0.75), ("f", -1.5)]
    got = caserun.run_case(oracle_lib, {"name": "gapgemm", "op": "nnc_hip_gap_gemm_nt", "tensors": tensors,
                                        "args": args, "outputs": ["out"]}, abi)["out"]
    mean = np.cumsum(x.reshape(n, c, h * w), axis=-1, dtype=F32)[..., -1] / F32(h * w)
    pooled = caserun.run_case(oracle_lib, {"name": "gap", "op": "nnc_avgpool2d",
                                           "tensors": {"x": x, "p": np.zeros((n, c, 1, 1), F32)},
                                           "args": [("t", "x"), ("t", "p"), ("i", h), ("i", w), ("i", h), ("i", w),
                                                    ("i", 0), ("i", 0)], "outputs": ["p"]}, abi)["p"]
    assert caserun.same_bits(pooled.reshape(n, c), mean.astype(F32))
    ref = mean.astype(np.float64) @ wt.astype(np.float64).T * 0.75
    if bias:
        ref = ref + -1.5 * tensors["c"].astype(np.float64)
    np.testing.assert_allclose(got, ref.astype(F32), rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("prog", range(8))
def test_oracle_fused_eltwise_composition(prog, oracle_lib, abi):
    """nnc_hip_fused_eltwise: each program equals its steps run as single
    nnc_* calls through temporaries (the oracle's own binary / unary / clip
    entry points, pinned against the reference above), bit for bit, also
    with the output written over an input."""
    from ew_cases import EW_PROGRAMS, ew_arrays, ew_case, ew_compose
    n_in, steps = EW_PROGRAMS[prog]
    xs = ew_arrays(n_in, 1031, 50 + prog)
    got = caserun.run_case(oracle_lib, ew_case(n_in, steps, xs), abi)["out"]
    assert caserun.same_bits(got, ew_compose(oracle_lib, abi, steps, xs))
    over = caserun.run_case(oracle_lib, ew_case(n_in, steps, xs, out_key="i0"), abi)["i0"]
    assert caserun.same_bits(over, got)


def test_oracle_fused_eltwise_closed_form(oracle_lib, abi):
    """The bandwidth chain's longer chain against numpy: add, relu, multiply
    and clip are exact in float32, sigmoid within a float32 ulp of float64."""
    from ew_cases import EW_PROGRAMS, ew_arrays, ew_case
    n_in, steps = EW_PROGRAMS[1]
    x, y, t = ew_arrays(n_in, 4096, 7)
    got = caserun.run_case(oracle_lib, ew_case(n_in, steps, [x, y, t]), abi)["out"]
    s = x + y
    r = np.where(s > 0, s, F32(0)) * x
    c = np.minimum(np.maximum(r, F32(-6)), F32(6)).astype(np.float64)
    ref = 1.0 / (1.0 + np.exp(-c)) + t.astype(np.float64)
    np.testing.assert_allclose(got, ref.astype(F32), rtol=2e-7, atol=2e-7)


@pytest.mark.parametrize("shape,axis,d", [((2, 4, 16, 16), -1, 2.0), ((3, 7), -1, -0.7), ((2, 5, 3), 1, 0.35)])
def test_oracle_scaled_softmax_composition(shape, axis, d, oracle_lib, abi):
    """nnc_hip_scaled_softmax: the oracle's nnc_div by the one-element
    divisor into a temporary, then its nnc_softmax (both pinned above), bit
    for bit; and within float32 rounding of float64 numpy softmax(x / d)
    (a negative divisor flips which element is the row maximum)."""
    rng = np.random.default_rng(4)
    x = (3 * rng.standard_normal(shape)).astype(F32)
    dv = np.array([d], F32)
    got = caserun.run_case(oracle_lib, {"name": "ssm", "op": "nnc_hip_scaled_softmax",
                                        "tensors": {"x": x, "d": dv, "out": np.zeros_like(x)},
                                        "args": [("t", "x"), ("t", "d"), ("t", "out"), ("i", axis)],
                                        "outputs": ["out"]}, abi)["out"]
    q = caserun.run_case(oracle_lib, {"name": "div", "op": "nnc_div", "tensors": {"x": x, "d": dv, "q": np.zeros_like(x)},
                                      "args": [("t", "x"), ("t", "d"), ("t", "q")], "outputs": ["q"]}, abi)["q"]
    want = caserun.run_case(oracle_lib, {"name": "sm", "op": "nnc_softmax", "tensors": {"q": q, "out": np.zeros_like(x)},
                                         "args": [("t", "q"), ("t", "out"), ("i", axis)], "outputs": ["out"]}, abi)["out"]
    assert caserun.same_bits(got, want)
    z = x.astype(np.float64) / float(dv[0])
    e = np.exp(z - z.max(axis=axis, keepdims=True))
    np.testing.assert_allclose(got, e / e.sum(axis=axis, keepdims=True), rtol=2e-6, atol=1e-7)


@pytest.mark.parametrize("rows,W,col0,view,perm", [(12, 24, 8, (3, 4, 2, 4), (0, 2, 1, 3)),
                                                   (12, 24, 16, (3, 4, 2, 4), (0, 2, 3, 1)),
                                                   (5, 7, 0, (5, 3), (1, 0))])
def test_oracle_transpose_slice(rows, W, col0, view, perm, oracle_lib, abi):
    """nnc_hip_transpose_slice: columns [col0, col0 + width) of every row,
    reshaped to the view and permuted - numpy's slice, reshape and
    transpose, exactly."""
    width = int(np.prod(view)) // rows
    x = np.arange(rows * W, dtype=F32).reshape(rows, W) * F32(0.5) - F32(3)
    want = np.ascontiguousarray(x[:, col0:col0 + width].reshape(view).transpose(perm))
    got = caserun.run_case(oracle_lib, {"name": "ts", "op": "nnc_hip_transpose_slice",
                                        "tensors": {"x": x, "out": np.zeros_like(want)},
                                        "args": [("t", "x"), ("t", "out"), ("i64", list(perm)), ("i", len(perm)),
                                                 ("i", col0), ("i", width)], "outputs": ["out"]}, abi)["out"]
    assert got.tobytes() == want.tobytes()


@pytest.mark.parametrize("shape,axis", [((3, 5, 256), -1), ((2, 6, 4, 3), 1)])
def test_oracle_add_layernorm_composition(shape, axis, oracle_lib, abi):
    """nnc_hip_add_layernorm: the oracle's nnc_add into a temporary, then its
    nnc_layernorm (both pinned above), bit for bit; and within float32
    rounding of float64 numpy (two-pass mean and variance over [axis:])."""
    rng = np.random.default_rng(3)
    a, b = (rng.standard_normal(shape).astype(F32) for _ in range(2))
    ax = axis % len(shape)
    n = shape[ax]
    g, bb = (1 + 0.1 * rng.standard_normal(n)).astype(F32), (0.1 * rng.standard_normal(n)).astype(F32)
    args = [("t", "g"), ("t", "bb"), ("t", "out"), ("i", axis), ("f", 1e-5)]
    got = caserun.run_case(oracle_lib, {"name": "addln", "op": "nnc_hip_add_layernorm",
                                        "tensors": {"a": a, "b": b, "g": g, "bb": bb, "out": np.zeros_like(a)},
                                        "args": [("t", "a"), ("t", "b")] + args, "outputs": ["out"]}, abi)["out"]
    s = caserun.run_case(oracle_lib, {"name": "add", "op": "nnc_add", "tensors": {"a": a, "b": b, "s": np.zeros_like(a)},
                                      "args": [("t", "a"), ("t", "b"), ("t", "s")], "outputs": ["s"]}, abi)["s"]
    want = caserun.run_case(oracle_lib, {"name": "ln", "op": "nnc_layernorm",
                                         "tensors": {"s": s, "g": g, "bb": bb, "out": np.zeros_like(a)},
                                         "args": [("t", "s")] + args, "outputs": ["out"]}, abi)["out"]
    assert caserun.same_bits(got, want)
    x = (a + b).astype(np.float64).reshape(int(np.prod(shape[:ax])), -1)
    mean = x.mean(axis=1, keepdims=True)
    var = ((x - mean) ** 2).mean(axis=1, keepdims=True)
    inner = int(np.prod(shape[ax + 1:]))
    ref = (x - mean) / np.sqrt(var + 1e-5) * np.repeat(g, inner) + np.repeat(bb, inner)
    np.testing.assert_allclose(got.reshape(ref.shape), ref, rtol=1e-4, atol=1e-5)


def attention_f64(qkv, d, batch, seq, heads, dh, q_col, k_col, v_col):
    """Multi-head attention in float64: softmax(Q K^T / d) V per batch and
    head, heads merged along the columns."""
    x = qkv.astype(np.float64).reshape(batch, seq, -1)
    out = np.zeros((batch, seq, heads * dh))
    for h in range(heads):
        q, k, v = (x[:, :, c + h * dh:c + (h + 1) * dh] for c in (q_col, k_col, v_col))
        s = q @ k.transpose(0, 2, 1) / d
        e = np.exp(s - s.max(axis=-1, keepdims=True))
        out[:, :, h * dh:(h + 1) * dh] = (e / e.sum(axis=-1, keepdims=True)) @ v
    return out.reshape(batch * seq, heads * dh)


def attention_case(rng, batch, seq, heads, dh, cols, d, extra=0):
    """nnc_hip_attention case: qkv rows of 3 * heads * dh (+ extra) floats."""
    ld = 3 * heads * dh + extra
    qkv = (rng.standard_normal((batch * seq, ld)) * 0.5).astype(F32)
    return {"name": "attn", "op": "nnc_hip_attention",
            "tensors": {"qkv": qkv, "d": np.array([d], F32), "out": np.zeros((batch * seq, heads * dh), F32)},
            "args": [("t", "qkv"), ("t", "d"), ("t", "out")] + [("i", v) for v in (batch, seq, heads, dh, *cols)],
            "outputs": ["out"]}


@pytest.mark.parametrize("batch,seq,heads,dh,cols,d,extra", [
    (2, 32, 2, 32, (0, 64, 128), 5.65, 0),      # two batches, two heads
    (1, 128, 4, 64, (0, 256, 512), 8.0, 0),     # the encoder's head shape
    (3, 64, 1, 64, (128, 0, 64), -1.5, 4),      # Q after K and V, a negative divisor, a wider row
])
def test_oracle_attention_composition(batch, seq, heads, dh, cols, d, extra, oracle_lib, abi):
    """nnc_hip_attention: per batch and head the oracle's nnc_matmul of Q and
    K^T, nnc_div, nnc_softmax over the keys and nnc_matmul with V (pinned
    above) on two-dimensional operands copied out of the qkv rows, merged
    back by head - within float32 rounding of float64 multi-head attention
    (a wrong column block, K not transposed, a product instead of the
    division or a softmax over the queries all fail it)."""
    case = attention_case(np.random.default_rng(9), batch, seq, heads, dh, cols, d, extra)
    got = caserun.run_case(oracle_lib, case, abi)["out"]
    ref = attention_f64(case["tensors"]["qkv"], d, batch, seq, heads, dh, *cols)
    np.testing.assert_allclose(got, ref, rtol=1e-5, atol=1e-6)
