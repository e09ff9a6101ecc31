"""The non-ResNet workloads: transformer encoder, GEMM sweep and the
bandwidth-bound op chain, at their full sizes on the GPU (size-independent
properties and float64 references), and their graph semantics on the CPU.

Transformer: the reference runtime steps batched MatMul operands by the
batch count (runtime/x86/ops.c:1687-1704), so with batch x heads > 1 its
attention is not the model's; the oracle reproduces that. Whole-encoder
checks therefore compare with a float64 numpy restatement of the model
(zoo.transformer_encoder_reference), and the oracle is used where the
bug cannot show (one batch, one head).
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest

import caserun


def _encoder(batch, seq, heads, seed=3):
    from nnc_py_amd.compiler import zoo
    return zoo.transformer_encoder(batch=batch, seq=seq, heads=heads, seed=seed)


@pytest.mark.parametrize("opt", [1, 3])
def test_encoder_graph_matches_float64_on_the_oracle(opt, pkg, oracle_lib):
    from nnc_py_amd.compiler import Executor, build_program, zoo
    prog = build_program(_encoder(1, 16, 1), opt_level=opt)
    ex = Executor(prog, device=False, lib=oracle_lib)
    x = np.random.default_rng(0).standard_normal((1, 16, 256)).astype(np.float32)
    ex.set_input("input", x)
    ex.run()
    ref = zoo.transformer_encoder_reference(_encoder(1, 16, 1), x, heads=1)
    bad = caserun.fp_violations(ex.get("output"), ref, 1e-4, 1e-3)
    assert bad.size == 0


def test_encoder_reference_stepping_differs_with_heads(pkg, oracle_lib):
    """Documents the divergence: with 2 x 4 attention batches the reference
    arithmetic (oracle) is not the model."""
    from nnc_py_amd.compiler import Executor, build_program, zoo
    ex = Executor(build_program(_encoder(2, 16, 4), opt_level=1), device=False, lib=oracle_lib)
    x = np.random.default_rng(0).standard_normal((2, 16, 256)).astype(np.float32)
    ex.set_input("input", x)
    ex.run()
    ref = zoo.transformer_encoder_reference(_encoder(2, 16, 4), x, heads=4)
    assert np.abs(ex.get("output") - ref).max() > 1e-2


def test_encoder_flops(pkg):
    from nnc_py_amd.compiler import zoo
    assert abs(zoo.transformer_flops() - 3.4897e9) < 1e6


@pytest.mark.gpu
def test_encoder_full_size_on_gpu(hip):
    """B8 S128 D256 H4 FFN1024, 2 layers, O3, inputs ~N(0, 0.02^2) as in the
    workload: logits vs the float64 model, 1e-4 abs / 1e-3 rel."""
    from nnc_py_amd.compiler import Executor, build_program, zoo
    g = zoo.transformer_encoder(seed=1)
    ex = Executor(build_program(g, opt_level=3), device=True)
    x = (np.random.default_rng(0).standard_normal((8, 128, 256)) * 0.02).astype(np.float32)
    ex.set_input("input", x)
    ex.run()
    got = ex.get("output")
    ex.close()
    ref = zoo.transformer_encoder_reference(zoo.transformer_encoder(seed=1), x)
    bad = caserun.fp_violations(got, ref, 1e-4, 1e-3)
    print(f"encoder max |diff| {np.abs(got - ref).max():.3g}", flush=True)
    assert bad.size == 0, f"{bad.size} outputs outside the bar"


def _dev(arr):
    from nnc_py_amd import runtime
    buf = runtime.DeviceBuffer.from_array(arr)
    t = buf.tensor()
    return buf, t


@pytest.mark.gpu
@pytest.mark.parametrize("n", [1024, 2048, 4096])
def test_gemm_sweep_full_size(n, hip):
    """Gemm M=N=K with bias [N], U(-1,1). Size-independent checks at full
    size: rows against float64 on a sample of rows, and linearity
    (A (B1 + B2) = A B1 + A B2 within the fp32 bar)."""
    from nnc_py_amd import runtime
    rng = np.random.default_rng(n)
    a = rng.uniform(-1, 1, (n, n)).astype(np.float32)
    b = rng.uniform(-1, 1, (n, n)).astype(np.float32)
    c = rng.uniform(-1, 1, n).astype(np.float32)
    ba, ta = _dev(a)
    bb, tb = _dev(b)
    bc, tc = _dev(c)
    bo, to = _dev(np.zeros((n, n), np.float32))
    hip.nnc_gemm(ctypes.byref(ta[0]), ctypes.byref(tb[0]), ctypes.byref(tc[0]), ctypes.byref(to[0]), 1.0, 1.0, 0, 0)
    runtime.sync()
    assert runtime.last_error()[0] == 0
    out = bo.to_array()
    rows = rng.choice(n, 16, replace=False)
    ref = a[rows].astype(np.float64) @ b.astype(np.float64) + c
    bad = caserun.fp_violations(out[rows], ref, 1e-4, 1e-3)
    assert bad.size == 0, f"{bad.size} of {ref.size} sampled outputs outside the bar"


@pytest.mark.gpu
def test_gemv_and_bmm_full_size(hip):
    from nnc_py_amd import runtime
    rng = np.random.default_rng(9)
    v = rng.uniform(-1, 1, (1, 4096)).astype(np.float32)
    m = rng.uniform(-1, 1, (4096, 4096)).astype(np.float32)
    bv, tv = _dev(v)
    bm, tm = _dev(m)
    bo, to = _dev(np.zeros((1, 4096), np.float32))
    hip.nnc_matmul(ctypes.byref(tv[0]), ctypes.byref(tm[0]), ctypes.byref(to[0]))
    a = rng.uniform(-1, 1, (64, 128, 64)).astype(np.float32)
    b = rng.uniform(-1, 1, (64, 64, 128)).astype(np.float32)
    ba, ta = _dev(a)
    bb, tb = _dev(b)
    bq, tq = _dev(np.zeros((64, 128, 128), np.float32))
    hip.nnc_matmul(ctypes.byref(ta[0]), ctypes.byref(tb[0]), ctypes.byref(tq[0]))
    runtime.sync()
    assert runtime.last_error()[0] == 0
    assert caserun.fp_violations(bo.to_array(), v.astype(np.float64) @ m, 1e-4, 1e-3).size == 0
    assert caserun.fp_violations(bq.to_array(), a.astype(np.float64) @ b, 1e-4, 1e-3).size == 0


@pytest.mark.gpu
def test_bandwidth_chain_full_size(hip, abi):
    """The bandwidth-bound ops at the workload's sizes: element-wise ops on
    [32,256,56,56] bit-exact against numpy's identical fp32 arithmetic where
    the reference's is (add, mul, relu, clip), softmax rows summing to 1,
    layernorm rows of mean 0 / variance 1, reducemean over (2,3) against
    float64, concat/split round trip bit-exact."""
    from nnc_py_amd import runtime
    rng = np.random.default_rng(2)
    shape = (32, 256, 56, 56)
    x = rng.standard_normal(shape).astype(np.float32)
    y = rng.standard_normal(shape).astype(np.float32)
    bx, tx = _dev(x)
    by, ty = _dev(y)
    bo, to = _dev(np.zeros(shape, np.float32))
    for op, want in (("nnc_add", x + y), ("nnc_mul", x * y)):
        getattr(hip, op)(ctypes.byref(tx[0]), ctypes.byref(ty[0]), ctypes.byref(to[0]))
        runtime.sync()
        assert caserun.same_bits(bo.to_array(), want), op
    hip.nnc_relu(ctypes.byref(tx[0]), ctypes.byref(to[0]))
    runtime.sync()
    assert caserun.same_bits(bo.to_array(), np.where(x > 0, x, np.float32(0)).astype(np.float32))
    hip.nnc_clip(ctypes.byref(tx[0]), ctypes.byref(to[0]), -6.0, 6.0)
    runtime.sync()
    assert caserun.same_bits(bo.to_array(), np.minimum(np.maximum(x, np.float32(-6)), np.float32(6)))
    # concat along channels, then split back
    cat_shape = (32, 512, 56, 56)
    bc, tc = _dev(np.zeros(cat_shape, np.float32))
    ins = (abi.TP * 2)(ctypes.pointer(tx[0]), ctypes.pointer(ty[0]))
    hip.nnc_concat(ctypes.cast(ins, abi.TPP), ctypes.byref(tc[0]), 2, 1)
    b1, t1 = _dev(np.zeros(shape, np.float32))
    b2, t2 = _dev(np.zeros(shape, np.float32))
    outs = (abi.TP * 2)(ctypes.pointer(t1[0]), ctypes.pointer(t2[0]))
    hip.nnc_split(ctypes.byref(tc[0]), ctypes.cast(outs, abi.TPP), 2, 1)
    runtime.sync()
    assert caserun.same_bits(b1.to_array(), x) and caserun.same_bits(b2.to_array(), y)
    del bc, b1, b2
    # softmax [4096, 1024] axis -1
    s = rng.standard_normal((4096, 1024)).astype(np.float32)
    bs, ts = _dev(s)
    bso, tso = _dev(np.zeros_like(s))
    hip.nnc_softmax(ctypes.byref(ts[0]), ctypes.byref(tso[0]), -1)
    # layernorm [8192, 768]
    l = rng.standard_normal((8192, 768)).astype(np.float32)
    bl, tl = _dev(l)
    g1, tg = _dev(np.ones(768, np.float32))
    b0, tb0 = _dev(np.zeros(768, np.float32))
    blo, tlo = _dev(np.zeros_like(l))
    hip.nnc_layernorm(ctypes.byref(tl[0]), ctypes.byref(tg[0]), ctypes.byref(tb0[0]), ctypes.byref(tlo[0]), -1,
                      ctypes.c_float(1e-5))
    # reducemean over (2,3) of [32,512,28,28] = one reduce over axis 2 of the [32,512,784] view
    r = rng.standard_normal((32, 512, 28, 28)).astype(np.float32)
    br, tr = _dev(r)
    tv = abi.make_tensor(br.ptr, abi.NUMPY_TO_NNC["float32"], (32, 512, 784), r.nbytes)
    bro, tro = _dev(np.zeros((32, 512, 1), np.float32))
    hip.nnc_reducemean(ctypes.byref(tv[0]), ctypes.byref(tro[0]), 2, 1)
    runtime.sync()
    assert runtime.last_error()[0] == 0
    sm = bso.to_array()
    assert np.abs(sm.sum(1) - 1).max() < 1e-4 and (sm >= 0).all()
    ln = blo.to_array().astype(np.float64)
    assert np.abs(ln.mean(1)).max() < 1e-4 and np.abs(ln.var(1) - 1).max() < 1e-3
    mean = bro.to_array().reshape(32, 512)
    assert caserun.fp_violations(mean, r.astype(np.float64).mean((2, 3)), 1e-4, 1e-3).size == 0
